"""kd_gpt_kael_init (host code of the product library) against kael's own GPT constructor on the CPU
(reference src/nn/transformer.cpp:167-207 after manual_seed; oracle/_ref's kael): every parameter of
a small model, of config C4's char-GPT (seed 3) and of config C5's GPT-2 small (seed 4), bit for
bit. bench.py draws C4's and C5's weights this way, so its runs use the configs' own models."""
import numpy as np
import pytest

import kd
import support


@pytest.fixture(scope="module")
def cpu_kael():
    return support.load_ref("ref")


CONFIGS = {"small": ((11, 16, 2, 2, 8), 31), "c4": ((96, 128, 4, 4, 256), 3), "odd": ((37, 9, 3, 3, 12), 2**40 + 7),
           "c5": ((50257, 1024, 12, 12, 768), 4)}


@pytest.mark.parametrize("which", list(CONFIGS))
def test_parameters_equal_kaels(cpu_kael, which):
    (vocab, positions, layers, heads, dim), seed = CONFIGS[which]
    h = cpu_kael.ref_gpt_create(vocab, positions, layers, heads, dim, seed, 1)
    assert h, support.ref_error(cpu_kael)
    try:
        want = support.export_gpt_params(cpu_kael, h)
    finally:
        cpu_kael.ref_gpt_destroy(h)
    got = kd.kael_gpt_parameters(kd.Backend(), seed, vocab, positions, layers, heads, dim)
    assert [n for n, _ in got] == [n for n, _ in want]
    for (name, g), (_, w) in zip(got, want):
        assert g.shape == w.shape, name
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), name
    if got[0][1].size >= 10000:  # the token table holds N(0, 0.02) draws
        assert np.std(got[0][1]) == pytest.approx(0.02, rel=0.05)


def test_rejects_bad_configs():
    b = kd.Backend()
    total = kd.c_int64()
    bad = kd.GptConfig(11, 16, 2, 3, 8, 1, 0)  # 8 does not divide by 3 heads
    assert b.lib.kd_gpt_kael_init(kd.ctypes.byref(bad), 1, None, 0, kd.ctypes.byref(total)) == -1
    ok = kd.GptConfig(11, 16, 2, 2, 8, 1, 0)
    assert b.lib.kd_gpt_kael_init(kd.ctypes.byref(ok), 1, None, 0, kd.ctypes.byref(total)) == 0
    buf = np.zeros(total.value - 1, np.float32)
    assert b.lib.kd_gpt_kael_init(kd.ctypes.byref(ok), 1, buf.ctypes.data_as(kd.c_void_p), buf.size,
                                  kd.ctypes.byref(total)) == -1
