"""kd_matmul / kd_matmul_strided against the C oracle.

Shapes: the reference's CudaMatmul list (tests/test_cuda.cpp:324-341), batched / vector /
integer / transposed cases (:343-355), BASELINE config C1 (512^3, uniform[-1,1]) and the GPT-2
decode and char-GPT training shapes. f32 and f64 use the reference device
tolerance rtol = atol = 1e-4 (tests/test_cuda.cpp:40-43) against a double-accumulated product;
i64 is exact with wrapping.
"""
import numpy as np
import pytest

import kd
import support

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1, 1), (4, 4, 4), (5, 3, 9), (8, 16, 7), (33, 20, 65), (64, 1, 64), (1, 64, 1),
          (512, 512, 512), (1, 768, 2304), (1, 3072, 768), (16, 768, 768), (130, 257, 129),
          (1000, 768, 1), (300, 64, 3), (64, 784, 128), (256, 128, 768)]


def reference_product(a, b):
    return np.matmul(a.astype(np.float64), b.astype(np.float64))


def close(got, want, rtol=1e-4, atol=1e-4):
    err = np.abs(got.astype(np.float64) - want)
    bad = err > atol + rtol * np.abs(want)
    assert not bad.any(), f"{bad.sum()} elements off; worst {err.max()}"


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64], ids=["f32", "f64"])
@pytest.mark.parametrize("m,k,n", SHAPES, ids=[f"{m}x{k}x{n}" for m, k, n in SHAPES])
def test_matmul_matches(kdb, dtype, m, k, n):
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    npd = kd.NUMPY_DTYPE[dtype]
    a = rng.uniform(-1, 1, (m, k)).astype(npd)
    b = rng.uniform(-1, 1, (k, n)).astype(npd)
    da, db, dc = kdb.to_device(a), kdb.to_device(b), kdb.empty((m, n), npd)
    kdb.call("matmul", dtype, da.ptr, db.ptr, dc.ptr, kd.MatmulSizes(1, m, k, n))
    close(dc.numpy(), reference_product(a, b))


def kael_uniform_pm1(refdev, seed, *shapes):
    """Arrays drawn as the configs specify: manual_seed(seed), then rand(shape) * 2 - 1 for each
    shape in turn from kael's generator (reference src/random.cpp)."""
    sizes = [int(np.prod(s)) for s in shapes]
    flat = np.empty(sum(sizes), np.float32)
    assert refdev.ref_uniform_pm1(seed, flat.size, support.ptr(flat)) == 0, support.ref_error(refdev)
    out, at = [], 0
    for s, n in zip(shapes, sizes):
        out.append(flat[at:at + n].reshape(s).copy())
        at += n
    return out


def test_c1_config_matches_kael_cpu_order(kdb, oracle, refdev):
    """C1 as the config draws it (manual_seed(0); A, B = rand({512,512}) * 2 - 1), against the
    oracle's reference device order."""
    a, b = kael_uniform_pm1(refdev, 0, (512, 512), (512, 512))
    want = np.empty((512, 512), np.float32)
    sizes = kd.MatmulSizes(1, 512, 512, 512)
    assert oracle.oracle_matmul(kd.F32, support.ptr(a), support.ptr(b), support.ptr(want), sizes, 0) == 0
    da, db, dc = kdb.to_device(a), kdb.to_device(b), kdb.empty((512, 512), np.float32)
    kdb.call("matmul", kd.F32, da.ptr, db.ptr, dc.ptr, sizes)
    close(dc.numpy(), want.astype(np.float64))


def test_batched_and_integer(kdb, oracle):
    rng = np.random.default_rng(3)
    a = rng.normal(size=(6, 4, 5)).astype(np.float32)
    b = rng.normal(size=(6, 5, 6)).astype(np.float32)
    da, db, dc = kdb.to_device(a), kdb.to_device(b), kdb.empty((6, 4, 6), np.float32)
    kdb.call("matmul", kd.F32, da.ptr, db.ptr, dc.ptr, kd.MatmulSizes(6, 4, 5, 6))
    close(dc.numpy(), reference_product(a, b))
    i = rng.integers(-5, 5, (3, 6, 6)).astype(np.int64)
    i[0, 0, 0] = 2**62
    di, do = kdb.to_device(i), kdb.empty((3, 6, 6), np.int64)
    kdb.call("matmul", kd.I64, di.ptr, di.ptr, do.ptr, kd.MatmulSizes(3, 6, 6, 6))
    want = np.empty((3, 6, 6), np.int64)
    assert oracle.oracle_matmul(kd.I64, support.ptr(i), support.ptr(i), support.ptr(want), kd.MatmulSizes(3, 6, 6, 6), 0) == 0
    np.testing.assert_array_equal(do.numpy(), want)


def test_bool_is_rejected_and_empty_is_zero(kdb):
    x = kdb.to_device(np.ones(4, np.uint8))
    with pytest.raises(kd.KdError):
        kdb.call("matmul", kd.BOOL, x.ptr, x.ptr, x.ptr, kd.MatmulSizes(1, 2, 2, 1))
    out = kdb.to_device(np.full((3, 2), 9.0, np.float32))
    kdb.call("matmul", kd.F32, out.ptr, out.ptr, out.ptr, kd.MatmulSizes(1, 3, 0, 2))
    np.testing.assert_array_equal(out.numpy(), np.zeros((3, 2), np.float32))


# (batches, M, K, N, a strides, b strides): transposed / batch-broadcast operands read in place.
STRIDED = [
    ("wT", 1, 64, 256, 768, (0, 256, 1), (0, 1, 256)),       # x . W^T with W [768, 256] row-major
    ("aT", 1, 256, 128, 96, (0, 1, 256), (0, 96, 1)),         # X^T . g
    ("both", 1, 130, 70, 200, (0, 1, 130), (0, 1, 70)),
    ("bcast", 4, 64, 128, 192, (64 * 128, 128, 1), (0, 1, 128)),  # batch-broadcast W^T
    ("decode", 1, 1, 768, 2304, (0, 768, 1), (0, 1, 768)),
    ("generic", 2, 33, 17, 40, (17 * 33 * 2, 1, 33 * 2), (0, 40 * 3, 3)),
]


@pytest.mark.parametrize("case", STRIDED, ids=[c[0] for c in STRIDED])
def test_strided_operands(kdb, oracle, case):
    name, batches, m, k, n, sa, sb = case
    rng = np.random.default_rng(len(name))

    def extent(shape, st):
        return 1 + sum((s - 1) * t for s, t in zip(shape, st))

    a_store = rng.uniform(-1, 1, extent((batches, m, k), sa)).astype(np.float32)
    b_store = rng.uniform(-1, 1, extent((batches, k, n), sb)).astype(np.float32)
    so = (m * n, n, 1)
    strides = kd.MatmulStrides()
    for i in range(3):
        strides.a[i], strides.b[i], strides.out[i] = sa[i], sb[i], so[i]
    sizes = kd.MatmulSizes(batches, m, k, n)
    want = np.empty((batches, m, n), np.float32)
    assert oracle.oracle_matmul_strided(kd.F32, support.ptr(a_store), support.ptr(b_store), support.ptr(want),
                                        sizes, strides) == 0
    da, db, dc = kdb.to_device(a_store), kdb.to_device(b_store), kdb.empty((batches, m, n), np.float32)
    kdb.call("matmul_strided", kd.F32, da.ptr, db.ptr, dc.ptr, sizes, strides)
    close(dc.numpy(), want.astype(np.float64))


def _strided_product(kdb, a_store, b_store, batches, m, k, n, sa, sb):
    strides = kd.MatmulStrides()
    so = (m * n, n, 1)
    for i in range(3):
        strides.a[i], strides.b[i], strides.out[i] = sa[i], sb[i], so[i]
    da, db, dc = kdb.to_device(a_store), kdb.to_device(b_store), kdb.empty((batches, m, n), np.float32)
    kdb.call("matmul_strided", kd.F32, da.ptr, db.ptr, dc.ptr, kd.MatmulSizes(batches, m, k, n), strides)
    return dc.numpy()


@pytest.mark.parametrize("a_t,b_t", [(True, False), (False, True), (True, True)], ids=["aT", "bT", "both"])
def test_transposed_whole_tiles_equal_row_major(kdb, a_t, b_t):
    """A and/or B read in place through transposed views, whole 128x128 tiles and enough of them
    to skip the small-product path (3 x 1024x256x1024): the product runs on the kernel that loads
    a transposed operand as 4x4 blocks and writes them transposed into the same LDS tiles the
    row-major kernel fills, with the same MFMA order, so it must equal bit for bit the row-major
    product of the materialized operands (reference src/autograd/functions_linalg.cpp:37,44 and
    src/nn/layers.cpp:43 issue X^T . g and x . W^T)."""
    batches, m, k, n = 3, 1024, 256, 1024
    rng = np.random.default_rng(44 + 2 * a_t + b_t)
    a = rng.uniform(-1, 1, (batches, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (batches, k, n)).astype(np.float32)
    a_store = np.ascontiguousarray(np.transpose(a, (0, 2, 1))) if a_t else a
    b_store = np.ascontiguousarray(np.transpose(b, (0, 2, 1))) if b_t else b
    sa = (k * m, 1, m) if a_t else (m * k, k, 1)
    sb = (k * n, 1, k) if b_t else (k * n, n, 1)
    got = _strided_product(kdb, a_store, b_store, batches, m, k, n, sa, sb)
    da, db, dc = kdb.to_device(a), kdb.to_device(b), kdb.empty((batches, m, n), np.float32)
    kdb.call("matmul", kd.F32, da.ptr, db.ptr, dc.ptr, kd.MatmulSizes(batches, m, k, n))
    np.testing.assert_array_equal(got, dc.numpy())
    close(got, np.matmul(a.astype(np.float64), b.astype(np.float64)))


def test_weight_gradient_shape_of_c4(kdb):
    """C4's Linear weight gradient X^T . g with X [4096 tokens, 256] and g [4096, 768] read in
    place (M 256, K 4096, N 768: whole tiles, K too long for the small-product path). At K = 4096
    an element's f32 error scales with its sum of |a||b|, so the check is the GPT-2 logits rule:
    within 1e-4 of the largest |element| of the float64 product."""
    m, k, n = 256, 4096, 768
    rng = np.random.default_rng(45)
    x = rng.uniform(-1, 1, (k, m)).astype(np.float32)
    g = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    got = _strided_product(kdb, x, g, 1, m, k, n, (0, 1, m), (0, n, 1))[0]
    want = np.matmul(x.T.astype(np.float64), g.astype(np.float64))
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))


@pytest.mark.parametrize("batches,k,b_t", [(32, 256, True), (32, 1024, True), (32, 1024, False), (1, 512, True)],
                         ids=["proj-WT", "fc2-WT", "fc2-W", "flat-WT"])
def test_linear_forward_shapes_of_c4(kdb, batches, k, b_t):
    """kael's Linear forward x . W^T at C4's narrow outputs (x [32, 128, K], W [256, K] shared by
    every batch item, reference src/nn/layers.cpp:43): 64 output tiles, so the batch folds into M
    and K is split over the device, the partial products added in split order. Checked against the
    float64 product within 1e-4 of its largest |element| (the GPT-2 logits rule), and run twice to
    check that the result is deterministic."""
    m, n = 128 * 32 // batches, 256
    rng = np.random.default_rng(46 + k + b_t)
    x = rng.uniform(-1, 1, (batches, m, k)).astype(np.float32)
    w = rng.uniform(-1, 1, (n, k)).astype(np.float32)  # W^T is [k, n]
    b_store = w if b_t else np.ascontiguousarray(w.T)
    sb = (0, 1, k) if b_t else (0, n, 1)
    got = _strided_product(kdb, x, b_store, batches, m, k, n, (m * k, k, 1), sb)
    again = _strided_product(kdb, x, b_store, batches, m, k, n, (m * k, k, 1), sb)
    np.testing.assert_array_equal(got, again)
    want = np.matmul(x.astype(np.float64), w.T.astype(np.float64))
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))


def test_64_tiles_equal_128_tiles(kdb):
    """3 batches of 1024 x 256 x 1024 have 192 128x128 tiles, fewer than the 256 CUs, and run on
    64x64 tiles; 4 batches have 256 and stay on 128x128 tiles. Each batch item's product is the same
    computation either way: the same (k, k + 4) MFMA pairs in the same K order, so the first three
    items must agree bit for bit."""
    m, k, n = 1024, 256, 1024
    rng = np.random.default_rng(51)
    a = rng.uniform(-1, 1, (4, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (4, k, n)).astype(np.float32)
    outs = []
    for batches in (3, 4):
        da, db = kdb.to_device(a[:batches]), kdb.to_device(b[:batches])
        dc = kdb.empty((batches, m, n), np.float32)
        kdb.call("matmul", kd.F32, da.ptr, db.ptr, dc.ptr, kd.MatmulSizes(batches, m, k, n))
        outs.append(dc.numpy())
    np.testing.assert_array_equal(outs[0], outs[1][:3])
    close(outs[0], np.matmul(a[:3].astype(np.float64), b[:3].astype(np.float64)))


ATTENTION = [(128, 128, 128, 64), (128, 128, 64, 128), (128, 64, 128, 128), (8, 64, 32, 64)]


@pytest.mark.parametrize("batches,m,k,n", ATTENTION, ids=[f"{b}x{m}x{k}x{n}" for b, m, k, n in ATTENTION])
def test_attention_shaped_batches(kdb, batches, m, k, n):
    """The batched products of C4's attention (32 x 4 heads: Q.K^T with K = head_dim 64, P.V with
    N = 64, and their gradients, reference src/nn/transformer.cpp:103-139) on 64x64 tiles, and the
    smallest whole case (64 x 32 x 64)."""
    rng = np.random.default_rng(52 + m + k + n)
    a = rng.uniform(-1, 1, (batches, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (batches, k, n)).astype(np.float32)
    da, db, dc = kdb.to_device(a), kdb.to_device(b), kdb.empty((batches, m, n), np.float32)
    kdb.call("matmul", kd.F32, da.ptr, db.ptr, dc.ptr, kd.MatmulSizes(batches, m, k, n))
    close(dc.numpy(), np.matmul(a.astype(np.float64), b.astype(np.float64)))


@pytest.mark.parametrize("a_t,b_t", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["rows", "aT", "bT", "both"])
def test_64_tiles_with_transposed_operands(kdb, a_t, b_t):
    """M and N multiples of 64 but not of 128 (192 x 96 x 320, 4 batches), every operand layout:
    the 64x64 kernel's loaders (coalesced along each stored operand's contiguous dim, A^T written
    transposed into a swizzled tile) against the float64 product; all four layouts equal bit for
    bit (the same tiles, MFMA pairs and order)."""
    batches, m, k, n = 4, 192, 96, 320
    rng = np.random.default_rng(53)
    a = rng.uniform(-1, 1, (batches, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (batches, k, n)).astype(np.float32)
    a_store = np.ascontiguousarray(np.transpose(a, (0, 2, 1))) if a_t else a
    b_store = np.ascontiguousarray(np.transpose(b, (0, 2, 1))) if b_t else b
    sa = (k * m, 1, m) if a_t else (m * k, k, 1)
    sb = (k * n, 1, k) if b_t else (k * n, n, 1)
    got = _strided_product(kdb, a_store, b_store, batches, m, k, n, sa, sb)
    plain = _strided_product(kdb, a, b, batches, m, k, n, (m * k, k, 1), (k * n, n, 1))
    np.testing.assert_array_equal(got, plain)
    close(got, np.matmul(a.astype(np.float64), b.astype(np.float64)))


def test_split_k_on_64_tiles(kdb):
    """C4's narrowest weight gradient X^T . g (M = N = 256, K = 4096: 16 tiles of 64x64) splits K
    16 ways over the device and adds the partial products in split order: within 1e-4 of the
    largest |element| of the float64 product, and the same bits on a second run."""
    m, k, n = 256, 4096, 256
    rng = np.random.default_rng(54)
    x = rng.uniform(-1, 1, (k, m)).astype(np.float32)
    g = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    got = _strided_product(kdb, x, g, 1, m, k, n, (0, 1, m), (0, n, 1))[0]
    again = _strided_product(kdb, x, g, 1, m, k, n, (0, 1, m), (0, n, 1))[0]
    np.testing.assert_array_equal(got, again)
    want = np.matmul(x.T.astype(np.float64), g.astype(np.float64))
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))


@pytest.mark.parametrize("m, k, n, sa, sb", [
    (96, 4096, 256, (0, 1, 96), (0, 256, 1)),       # kael's tied LM-head weight gradient (A read transposed)
    (100, 1024, 128, (0, 1024, 1), (0, 128, 1)),    # ragged M on 64x64 tiles, A row-major
    (36, 2048, 64, (0, 1, 36), (0, 64, 1)),         # one ragged tile row, A read transposed
    (68, 96, 192, (0, 96, 1), (0, 1, 96)),          # ragged M, short K (no split), B read transposed
    (130, 3072, 70, (0, 3072, 1), (0, 1, 3072)),    # ragged M and N, B read transposed
    (33, 2560, 200, (0, 2, 67), (0, 200, 1)),       # generic A strides
], ids=["head_96x4096x256", "ragged_100x1024x128", "ragged_36x2048x64", "ragged_68x96x192", "ragged_130x3072x70",
        "generic_33x2560x200"])
def test_split_k_on_ragged_tiles(kdb, m, k, n, sa, sb):
    """Few ragged tiles with a long K: K split over the device (the splits in the kernel's batch
    slot; 64x64 tiles whose last tile row loads zeros past M and stores only rows below it when M
    is a multiple of 4 and N of 64, else the general kernel) and split_sum_kernel adding the
    partials in split order: within 1e-4 of the largest |element| of the float64 product, and the
    same bits on a second run."""
    rng = np.random.default_rng(m + k + n)

    def extent(shape, st):
        return 1 + sum((s - 1) * t for s, t in zip(shape, st))

    a_store = rng.uniform(-1, 1, extent((1, m, k), sa)).astype(np.float32)
    b_store = rng.uniform(-1, 1, extent((1, k, n), sb)).astype(np.float32)
    got = _strided_product(kdb, a_store, b_store, 1, m, k, n, sa, sb)[0]
    again = _strided_product(kdb, a_store, b_store, 1, m, k, n, sa, sb)[0]
    np.testing.assert_array_equal(got, again)
    a = np.lib.stride_tricks.as_strided(a_store, (m, k), (sa[1] * 4, sa[2] * 4)).astype(np.float64)
    b = np.lib.stride_tricks.as_strided(b_store, (k, n), (sb[1] * 4, sb[2] * 4)).astype(np.float64)
    want = a @ b
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))


def test_headline_4096_cubed(kdb, refdev, oracle):
    """The benchmark's headline product (row-major MFMA kernel, whole tiles) at its full size,
    inputs as bench.py draws them. At K = 4096 an element's f32 rounding error scales with its
    dot product's sum of |a||b| (~1024 here), not with the element itself, so elements near
    zero miss the small-shape rule 1e-4 + 1e-4 |y| by a few ulps of that sum in any f32
    product. Checks: within 1e-4 of the largest |element| of the float64 product (the rule of
    the GPT-2 logits), and within 8x the worst error of kael's own f32 CPU product of the same
    inputs (reference matmul_versions v6). Measured: device worst 3.6e-4 (one running f32 MFMA
    sum over K), kael CPU 6.6e-5 (its K blocking shortens the running sums), scale ~1e2."""
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, (4096, 4096)).astype(np.float32)
    b = rng.uniform(-1, 1, (4096, 4096)).astype(np.float32)
    da, db, dc = kdb.to_device(a), kdb.to_device(b), kdb.empty((4096, 4096), np.float32)
    kdb.call("matmul", kd.F32, da.ptr, db.ptr, dc.ptr, kd.MatmulSizes(1, 4096, 4096, 4096))
    got = dc.numpy().astype(np.float64)
    want = reference_product(a, b)
    refdev.ref_set_threads(min(16, max(1, __import__("os").cpu_count() or 1)))
    cpu = np.empty((4096, 4096), np.float32)
    assert refdev.ref_matmul(kd.F32, support.ptr(a), support.ptr(b), support.ptr(cpu), 1, 4096, 4096, 4096) == 0, \
        support.ref_error(refdev)
    err = np.abs(got - want)
    err_cpu = np.abs(cpu.astype(np.float64) - want)
    assert err.max() <= 1e-4 * np.abs(want).max(), f"worst {err.max()} vs scale {np.abs(want).max()}"
    assert err.max() <= 8 * err_cpu.max(), f"device worst {err.max()}, kael CPU worst {err_cpu.max()}"
    # The reference's device kernel (src/cuda/kernels.inl:136-177) keeps one running f32 sum per
    # element over k = 0 .. K-1, as this backend's MFMA accumulators do: on 64 sampled rows the
    # device's error must not exceed that order's (the oracle's restatement) by more than 1.5x.
    rows = np.random.default_rng(1).choice(4096, 64, replace=False)
    a_rows = np.ascontiguousarray(a[rows])
    order = np.empty((64, 4096), np.float32)
    assert oracle.oracle_matmul(kd.F32, support.ptr(a_rows), support.ptr(b), support.ptr(order),
                                kd.MatmulSizes(1, 64, 4096, 4096), 0) == 0
    err_rows = err[rows]
    err_order = np.abs(order.astype(np.float64) - want[rows])
    rms = lambda e: float(np.sqrt(np.mean(e * e)))  # noqa: E731
    print(f"\n4096^3 on 64 rows: device max {err_rows.max():.3e} rms {rms(err_rows):.3e}; reference device order "
          f"max {err_order.max():.3e} rms {rms(err_order):.3e}; kael CPU max {err_cpu.max():.3e}")
    assert err_rows.max() <= 1.5 * err_order.max()
    assert rms(err_rows) <= 1.5 * rms(err_order)


@pytest.mark.parametrize("batches,m,k,n", [(2, 384, 256, 512), (3, 128, 1024, 128)])
def test_batched_whole_tiles_with_split_k(kdb, batches, m, k, n):
    """Batched row-major products with few tiles: the row-major kernel splits K and sums the
    partials per batch."""
    rng = np.random.default_rng(m + k + n)
    a = rng.uniform(-1, 1, (batches, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (batches, k, n)).astype(np.float32)
    da, db, dc = kdb.to_device(a), kdb.to_device(b), kdb.empty((batches, m, n), np.float32)
    kdb.call("matmul", kd.F32, da.ptr, db.ptr, dc.ptr, kd.MatmulSizes(batches, m, k, n))
    close(dc.numpy(), reference_product(a, b))


def random_operand_strides(rng, batches, rows, cols, allow_broadcast):
    """Element strides (batch, row, col) of a random layout for a [batches, rows, cols] operand:
    row-major, column-major (a transposed view), stepped rows and columns, and, for inputs, a
    batch stride of 0 (one matrix broadcast to every batch). Returns (strides, storage length)."""
    kind = rng.integers(0, 4)
    step_r, step_c = (int(rng.integers(1, 3)), int(rng.integers(1, 3))) if kind == 2 else (1, 1)
    if kind == 1:  # column-major matrices
        st = [rows * cols, 1, rows]
    else:
        st = [rows * cols * step_r * step_c, cols * step_c * step_r, step_c]
    if allow_broadcast and batches > 1 and rng.random() < 0.3:
        st[0] = 0
    extent = 1 + (batches - 1) * st[0] + (rows - 1) * st[1] + (cols - 1) * st[2]
    return tuple(st), extent


DIMS = [1, 2, 3, 7, 16, 33, 64, 100, 128, 130, 257]


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64], ids=["f32", "f64"])
@pytest.mark.parametrize("block", range(4))
def test_random_strided_products(kdb, oracle, dtype, block):
    """60 seeded random products per dtype: sizes from 1 to 257 (whole and ragged tiles,
    skinny and row-dot shapes), every operand in a random layout, batch broadcast of either
    input, row- or column-major output; against the oracle's double-accumulated product."""
    npd = kd.NUMPY_DTYPE[dtype]
    for seed in range(block * 15, (block + 1) * 15):
        rng = np.random.default_rng(seed)
        batches = int(rng.integers(1, 4))
        m, k, n = (DIMS[int(rng.integers(0, len(DIMS)))] for _ in range(3))
        sa, la = random_operand_strides(rng, batches, m, k, True)
        sb, lb = random_operand_strides(rng, batches, k, n, True)
        so = (m * n, n, 1) if rng.random() < 0.7 else (m * n, 1, m)
        a_store = rng.uniform(-1, 1, la).astype(npd)
        b_store = rng.uniform(-1, 1, lb).astype(npd)
        strides = kd.MatmulStrides()
        for i in range(3):
            strides.a[i], strides.b[i], strides.out[i] = sa[i], sb[i], so[i]
        sizes = kd.MatmulSizes(batches, m, k, n)
        want = np.zeros(batches * m * n, npd)
        assert oracle.oracle_matmul_strided(dtype, support.ptr(a_store), support.ptr(b_store), support.ptr(want),
                                            sizes, strides) == 0
        da, db, dc = kdb.to_device(a_store), kdb.to_device(b_store), kdb.empty((batches * m * n,), npd)
        kdb.call("matmul_strided", dtype, da.ptr, db.ptr, dc.ptr, sizes, strides)
        try:
            close(dc.numpy(), want.astype(np.float64))
        except AssertionError as e:
            raise AssertionError(f"seed {seed}: {batches}x{m}x{k}x{n} a{sa} b{sb} out{so}: {e}") from None


def heads_call(kdb, dtype, a_store, b_store, out_len, sizes, sa, sb, so, heads, ha, hb, ho):
    strides = kd.MatmulStrides()
    for i in range(3):
        strides.a[i], strides.b[i], strides.out[i] = sa[i], sb[i], so[i]
    h = kd.MatmulHeads(heads, ha, hb, ho)
    npd = kd.NUMPY_DTYPE[dtype]
    da, db, dc = kdb.to_device(a_store), kdb.to_device(b_store), kdb.empty((out_len,), npd)
    kdb.call("matmul_strided_heads", dtype, da.ptr, db.ptr, dc.ptr, sizes, strides, h)
    return dc.numpy(), strides, h


def test_attention_head_views_equal_copied_operands(kdb, oracle):
    """C4's attention products over views of the fused qkv projection [B, T, 3, H, D] and of the
    output gradient [B, T, H, D] (B 32, T 128, H 4, D 64): Q.K^T, P.V, dY.V^T, P^T.dY and dS.K,
    read in place through two-level batch strides, against the same products of the views copied
    to contiguous tensors (the path kael takes without these strides): the same bits, and the
    oracle within the device tolerance."""
    B, T, H, D = 32, 128, 4, 64
    C = H * D
    rng = np.random.default_rng(11)
    qkv = rng.uniform(-1, 1, (B, T, 3, H, D)).astype(np.float32)
    dy = rng.uniform(-1, 1, (B, T, H, D)).astype(np.float32)
    p = rng.uniform(0, 1, (B, H, T, T)).astype(np.float32)
    q_v = (T * 3 * C, D, 3 * C, 1)          # outer, head, row, column strides of q[b, h] = qkv[b, :, 0, h, :]
    kT = (T * 3 * C, D, 1, 3 * C)           # k[b, h]^T
    k_v = (T * 3 * C, D, 3 * C, 1)
    dy_v = (T * C, D, C, 1)
    p_v, pT = (H * T * T, T * T, T, 1), (H * T * T, T * T, 1, T)
    views = {"q": (qkv, 0, q_v, (T, D)), "kT": (qkv, C, kT, (D, T)), "k": (qkv, C, k_v, (T, D)),
             "v": (qkv, 2 * C, k_v, (T, D)), "vT": (qkv, 2 * C, kT, (D, T)), "dy": (dy, 0, dy_v, (T, D)),
             "p": (p, 0, p_v, (T, T)), "pT": (p, 0, pT, (T, T))}

    def dense(name):
        store, off, (so_, sh, sr, sc), (r, c) = views[name]
        flat = store.ravel()[off:]
        return np.lib.stride_tricks.as_strided(flat, (B, H, r, c), tuple(4 * x for x in (so_, sh, sr, sc))).copy()

    for left, right in [("q", "kT"), ("p", "v"), ("dy", "vT"), ("pT", "dy"), ("p", "k")]:
        la, lb = views[left], views[right]
        m, k = la[3]
        n = lb[3][1]
        sizes = kd.MatmulSizes(B * H, m, k, n)
        so = (H * m * n, n, 1)
        a_store, b_store = la[0].ravel()[la[1]:].copy(), lb[0].ravel()[lb[1]:].copy()
        got, strides, h = heads_call(kdb, kd.F32, a_store, b_store, B * H * m * n, sizes, (la[2][0], la[2][2], la[2][3]),
                                     (lb[2][0], lb[2][2], lb[2][3]), so, H, la[2][1], lb[2][1], m * n)
        copied = _strided_product(kdb, dense(left).ravel(), dense(right).ravel(), B * H, m, k, n, (m * k, k, 1), (k * n, n, 1))
        np.testing.assert_array_equal(got, copied.ravel(), err_msg=f"{left}.{right}")
        want = np.empty(B * H * m * n, np.float32)
        assert oracle.oracle_matmul_strided_heads(kd.F32, support.ptr(a_store), support.ptr(b_store), support.ptr(want),
                                                  sizes, strides, h) == 0
        close(got, want.astype(np.float64))


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64], ids=["f32", "f64"])
def test_random_two_level_batches(kdb, oracle, dtype):
    """30 seeded products over random [outer, heads] batches: random row / column / head / outer
    strides (head dims interleaved with the rows, as attention's are, or blocked), ragged and whole
    tiles, f32 on every kernel family; against oracle_matmul_strided_heads."""
    npd = kd.NUMPY_DTYPE[dtype]
    for seed in range(30):
        rng = np.random.default_rng(1000 + seed)
        outer, heads = int(rng.integers(1, 4)), int(rng.integers(2, 5))
        m, k, n = (DIMS[int(rng.integers(0, len(DIMS)))] for _ in range(3))

        def operand(rows, cols):
            gap = int(rng.integers(0, 3))
            if rng.random() < 0.5:   # heads interleaved: [rows][heads][cols] (+ gap)
                st = (rows * (heads * cols + gap), cols, heads * cols + gap, 1)
            else:                    # transposed within the head: [heads][cols][rows]
                st = (heads * cols * (rows + gap), cols * (rows + gap), 1, rows + gap)
            extent = 1 + (outer - 1) * st[0] + (heads - 1) * st[1] + (rows - 1) * st[2] + (cols - 1) * st[3]
            return st, extent

        sa, la = operand(m, k)
        sb, lb = operand(k, n)
        a_store = rng.uniform(-1, 1, la).astype(npd)
        b_store = rng.uniform(-1, 1, lb).astype(npd)
        sizes = kd.MatmulSizes(outer * heads, m, k, n)
        so = (heads * m * n, n, 1)
        got, strides, h = heads_call(kdb, dtype, a_store, b_store, outer * heads * m * n, sizes, (sa[0], sa[2], sa[3]),
                                     (sb[0], sb[2], sb[3]), so, heads, sa[1], sb[1], m * n)
        want = np.zeros(outer * heads * m * n, npd)
        assert oracle.oracle_matmul_strided_heads(dtype, support.ptr(a_store), support.ptr(b_store), support.ptr(want),
                                                  sizes, strides, h) == 0
        try:
            close(got, want.astype(np.float64))
        except AssertionError as e:
            raise AssertionError(f"seed {seed}: {outer}x{heads} {m}x{k}x{n} a{sa} b{sb}: {e}") from None


def test_two_level_batches_reject_bad_heads(kdb):
    x = kdb.to_device(np.zeros(64, np.float32))
    strides = kd.MatmulStrides()
    for i, v in enumerate((16, 4, 1)):
        strides.a[i] = strides.b[i] = strides.out[i] = v
    for heads, batches in ((0, 2), (3, 4)):
        with pytest.raises(kd.KdError):
            kdb.call("matmul_strided_heads", kd.F32, x.ptr, x.ptr, x.ptr, kd.MatmulSizes(batches, 2, 2, 2), strides,
                     kd.MatmulHeads(heads, 8, 8, 8))


BIAS_CASES = [  # batches, m, k, n, a strides, b strides: kael's x . W^T shapes and every kernel family
    (32, 128, 256, 768, (128 * 256, 256, 1), (0, 1, 256)),      # t64 folded (C4 qkv)
    (32, 128, 256, 1024, (128 * 256, 256, 1), (0, 1, 256)),     # 128x128 transposed-B kernel (C4 fc1)
    (1, 4096, 4096, 256, (0, 4096, 1), (0, 1, 4096)),           # split K
    (1, 512, 512, 512, (0, 512, 1), (0, 512, 1)),               # row-major whole tiles / small kernel
    (1, 3, 768, 2304, (0, 768, 1), (0, 1, 768)),                # skinny (decode-shaped)
    (1, 64, 784, 128, (0, 784, 1), (0, 1, 784)),                # C3's first Linear
    (2, 33, 17, 3, (17 * 33, 17, 1), (0, 1, 17)),               # row-dot
    (2, 130, 70, 200, (130 * 70, 70, 1), (0, 1, 70)),           # ragged tiles, general kernel
    (1, 96, 4096, 256, (0, 1, 96), (0, 256, 1)),                # ragged tiles, general kernel split K
]


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64], ids=["f32", "f64", "i64"])
@pytest.mark.parametrize("case", BIAS_CASES, ids=[f"{c[0]}x{c[1]}x{c[2]}x{c[3]}" for c in BIAS_CASES])
def test_bias_epilogue_equals_product_then_add(kdb, oracle, dtype, case):
    """kd_matmul_strided_bias against kd_matmul_strided followed by a separate add of the bias
    broadcast over the rows (kael's product + bias): the same bits, since the product is the same
    kernel and the epilogue rounds the sum once; against the oracle within the device tolerance
    (exact for i64)."""
    batches, m, k, n, sa, sb = case
    if dtype != kd.F32 and m * n * k * batches > (1 << 28):
        pytest.skip("large shapes run for f32 only")
    npd = kd.NUMPY_DTYPE[dtype]
    rng = np.random.default_rng(batches * 3 + m + n)

    def extent(shape, st):
        return 1 + sum((s - 1) * t for s, t in zip(shape, st))

    if dtype == kd.I64:
        a_store = rng.integers(-9, 10, extent((batches, m, k), sa)).astype(npd)
        b_store = rng.integers(-9, 10, extent((batches, k, n), sb)).astype(npd)
        bias = rng.integers(-50, 50, n).astype(npd)
    else:
        a_store = rng.uniform(-1, 1, extent((batches, m, k), sa)).astype(npd)
        b_store = rng.uniform(-1, 1, extent((batches, k, n), sb)).astype(npd)
        bias = rng.uniform(-1, 1, n).astype(npd)
        bias[0] = -0.0
    so = (m * n, n, 1)
    strides = kd.MatmulStrides()
    for i in range(3):
        strides.a[i], strides.b[i], strides.out[i] = sa[i], sb[i], so[i]
    sizes = kd.MatmulSizes(batches, m, k, n)
    da, db, dbias = kdb.to_device(a_store), kdb.to_device(b_store), kdb.to_device(bias)
    fused, plain = kdb.empty((batches, m, n), npd), kdb.empty((batches, m, n), npd)
    kdb.call("matmul_strided_bias", dtype, da.ptr, db.ptr, fused.ptr, sizes, strides, dbias.ptr)
    kdb.call("matmul_strided", dtype, da.ptr, db.ptr, plain.ptr, sizes, strides)
    p = plain.numpy()
    if dtype == kd.I64:
        want_sum = (p.view(np.uint64) + bias.view(np.uint64)).view(np.int64)
    else:
        want_sum = p + bias  # one rounded add per element, as kael's add kernel
    got = fused.numpy()
    np.testing.assert_array_equal(got, want_sum)
    want = np.empty((batches, m, n), npd)
    assert oracle.oracle_matmul_strided_bias(dtype, support.ptr(a_store), support.ptr(b_store), support.ptr(want), sizes,
                                             strides, support.ptr(bias)) == 0
    if dtype == kd.I64:
        np.testing.assert_array_equal(got, want)
    else:
        close(got, want.astype(np.float64))


F64_CASES = [(1, 64, 16, 64), (1, 128, 256, 192), (3, 70, 33, 130), (2, 1, 5, 1), (1, 257, 1000, 65), (4, 64, 64, 64)]


@pytest.mark.parametrize("case", F64_CASES, ids=[f"{b}x{m}x{k}x{n}" for b, m, k, n in F64_CASES])
@pytest.mark.parametrize("layout", ["rowmajor", "transposed"])
def test_f64_on_the_matrix_cores(kdb, oracle, case, layout):
    """f64 products on v_mfma_f64_16x16x4f64 (whole and ragged tiles, batches, A and B read
    through transposed strides) against the oracle's sequential double sums: within 1e-13 of
    sum |a| |b| per element (the matrix cores accumulate four products per step in their own
    order). Also pins the instruction's lane layout: a wrong row / column assignment is far off."""
    batches, m, k, n = case
    rng = np.random.default_rng(m * 11 + n + k)
    if layout == "rowmajor":
        sa, sb = (m * k, k, 1), (k * n, n, 1)
    else:
        sa, sb = (m * k, 1, m), (k * n, 1, k)
    a = rng.uniform(-1, 1, batches * m * k)
    b = rng.uniform(-1, 1, batches * k * n)
    strides = kd.MatmulStrides()
    so = (m * n, n, 1)
    for i in range(3):
        strides.a[i], strides.b[i], strides.out[i] = sa[i], sb[i], so[i]
    sizes = kd.MatmulSizes(batches, m, k, n)
    want = np.empty(batches * m * n)
    assert oracle.oracle_matmul_strided(kd.F64, support.ptr(a), support.ptr(b), support.ptr(want), sizes, strides) == 0
    da, db, dc = kdb.to_device(a), kdb.to_device(b), kdb.empty((batches * m * n,), np.float64)
    kdb.call("matmul_strided", kd.F64, da.ptr, db.ptr, dc.ptr, sizes, strides)
    av = np.lib.stride_tricks.as_strided(a, (batches, m, k), tuple(8 * s for s in sa))
    bv = np.lib.stride_tricks.as_strided(b, (batches, k, n), tuple(8 * s for s in sb))
    scale = (np.abs(av) @ np.abs(bv)).ravel()
    assert np.all(np.abs(dc.numpy() - want) <= 1e-13 * scale + 1e-300)
