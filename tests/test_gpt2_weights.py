"""Hugging Face GPT-2 checkpoints into the decode engine's parameters (kd.gpt2_state_from_hf),
against kael's own load_gpt2_weights behaviour (reference src/nn/transformer.cpp:54-89,297-308
and its tests tests/test_transformer.cpp:286-329): names translated with or without the
`transformer.` prefix, Conv1D weights transposed, unknown entries ignored, a missing one an
error. The weights come from kael's GPT itself, so the round trip must be exact.
"""
import numpy as np
import pytest

import kd
import support


def tiny_expected():
    return dict(kd.gpt2_parameter_shapes(vocab_size=11, max_positions=16, layers=2, dimension=8))


@pytest.fixture
def kael_params(refdev):
    h = refdev.ref_gpt_create(11, 16, 2, 2, 8, 5, 1)
    assert h, support.ref_error(refdev)
    try:
        yield support.export_gpt_params(refdev, h)
    finally:
        refdev.ref_gpt_destroy(h)


def test_names_follow_the_reference_translation():
    assert kd.gpt2_name("transformer.h.1.attn.c_attn.weight") == "blocks.1.attn.qkv.weight"
    assert kd.gpt2_name("h.0.mlp.c_proj.bias") == "blocks.0.mlp.fc2.bias"
    assert kd.gpt2_name("h.10.ln_2.weight") == "blocks.10.ln2.weight"
    assert kd.gpt2_name("wte.weight") == "token_embedding.weight"
    assert kd.gpt2_name("transformer.wpe.weight") == "position_embedding.weight"
    assert kd.gpt2_name("ln_f.bias") == "ln_final.bias"
    assert kd.gpt2_name("lm_head.weight") == "lm_head.weight"  # not a kael parameter: ignored
    assert kd.gpt2_stored_transposed("blocks.0.mlp.fc1.weight")
    assert not kd.gpt2_stored_transposed("blocks.0.mlp.fc1.bias")
    assert not kd.gpt2_stored_transposed("token_embedding.weight")


@pytest.mark.parametrize("prefix", [True, False], ids=["transformer_prefix", "bare"])
def test_round_trip_through_a_safetensors_file(tmp_path, kael_params, prefix):
    from safetensors import safe_open
    from safetensors.numpy import save_file

    path = tmp_path / "model.safetensors"
    save_file(support.hf_gpt2_tensors(kael_params, prefix_blocks=prefix), str(path))
    with safe_open(str(path), framework="numpy") as f:
        state = kd.gpt2_state_from_hf({k: f.get_tensor(k) for k in f.keys()}, tiny_expected())
    assert set(state) == {n for n, _ in kael_params}
    for name, array in kael_params:
        np.testing.assert_array_equal(state[name], array, err_msg=name)


def test_missing_entries_are_reported(kael_params):
    hf = support.hf_gpt2_tensors(kael_params)
    del hf["transformer.h.1.mlp.c_fc.bias"]
    with pytest.raises(ValueError, match="missing"):
        kd.gpt2_state_from_hf(hf, tiny_expected())
    with pytest.raises(ValueError, match="missing"):
        kd.gpt2_state_from_hf({"wte.weight": np.zeros((11, 8), np.float32)}, tiny_expected())


def test_misshapen_entries_are_rejected(kael_params):
    hf = support.hf_gpt2_tensors(kael_params)
    hf["transformer.h.0.attn.c_attn.weight"] = hf["transformer.h.0.attn.c_attn.weight"].T.copy()  # not transposed
    with pytest.raises(ValueError, match="shape"):
        kd.gpt2_state_from_hf(hf, tiny_expected())
