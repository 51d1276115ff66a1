"""CPU tests of the drop-in boundary and the host logic (no GPU compute).

- The C-ABI library loads and exports every function include/nimbleml_hip.h declares,
  and the ctypes binding covers exactly that set.
- Host-side mirror of the reference API: parameter names, checkpoint round trip,
  the device weight layout (transpose / Q-K-V stacking), input validation and the
  error types the reference raises, and the "no device" failure.
"""
import os
import re

import numpy as np
import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "nimbleml_hip.h")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(nml_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    import ctypes

    from nimbleml_amd import _native

    declared = header_functions()
    assert len(declared) >= 30
    lib = ctypes.CDLL(_native.LIB_PATH)
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(_native.exported_symbols()) == declared


def test_no_device_is_a_clear_runtime_error():
    import nimbleml_amd as nm
    from nimbleml_amd import _native

    if _native.device_count() > 0:
        pytest.skip("a GPU is visible")
    m = nm.GPT(64, 16, 2, 1, 8)
    with pytest.raises(RuntimeError, match="no HIP device"):
        m.forward(np.zeros((1, 4), dtype=np.int64))


def test_parameter_names_match_reference_checkpoint_names():
    import nimbleml_amd as nm
    from oracle.weights import GPTConfig, param_shapes

    cfg = GPTConfig(40, 16, 4, 3, 12)
    m = nm.GPT(cfg.vocab_size, cfg.d_model, cfg.num_heads, cfg.num_layers, cfg.max_seq_len)
    got = {n: p.shape for n, p in nm.named_parameters(m)}
    want = dict(param_shapes(cfg))
    assert got == want
    # parameters() keeps the reference's order: token_emb, blocks, pos_emb, ln
    params = m.parameters()
    assert params[0] is m.token_emb.weights and params[-1] is m.ln.gamma


def test_save_load_roundtrip_and_mismatch(tmp_path):
    import nimbleml_amd as nm
    from oracle.weights import GPTConfig, make_weights

    cfg = GPTConfig(30, 8, 2, 2, 6)
    m = nm.GPT(30, 8, 2, 2, 6)
    w = make_weights(cfg, seed=3, rich=True)
    nm.load_arrays(m, w)
    p = tmp_path / "w.npz"
    nm.save(m, p)
    m2 = nm.GPT(30, 8, 2, 2, 6)
    nm.load(m2, p)
    for (n1, a), (n2, b) in zip(nm.named_parameters(m), nm.named_parameters(m2)):
        assert n1 == n2 and np.array_equal(a.data, b.data)
    bad = dict(w)
    bad.pop("ln.gamma")
    with pytest.raises(ValueError, match="missing"):
        nm.load_arrays(m, bad)


def test_device_layout_reproduces_reference_projections():
    """The uploaded (out, in) / stacked-QKV arrays give the reference's x @ W products."""
    import nimbleml_amd as nm
    from nimbleml_amd import _native as N
    from oracle.weights import GPTConfig, make_weights

    cfg = GPTConfig(30, 8, 2, 1, 6)
    m = nm.GPT(30, 8, 2, 1, 6)
    w = make_weights(cfg, seed=9, rich=True)
    nm.load_arrays(m, w)
    arrs = {(k, l): a for k, l, a in m._device_arrays()}
    x = np.random.default_rng(0).standard_normal((5, 8)).astype(np.float32)
    p = "blocks.layers.0."
    qkv = x @ arrs[(N.P_WQKV, 0)].T + arrs[(N.P_BQKV, 0)]
    want = np.concatenate([x @ w[p + f"mha.W_{c}.weights"] + w[p + f"mha.W_{c}.biases"]
                           for c in "qkv"], axis=1)
    assert np.allclose(qkv, want, atol=1e-6)
    assert np.allclose(x @ arrs[(N.P_WO, 0)].T, x @ w[p + "mha.W_o.weights"], atol=1e-6)
    h = np.random.default_rng(1).standard_normal((5, 32)).astype(np.float32)
    assert np.allclose(x @ arrs[(N.P_W1, 0)].T, x @ w[p + "ffn.dense1.weights"], atol=1e-6)
    assert np.allclose(h @ arrs[(N.P_W2, 0)].T, h @ w[p + "ffn.dense2.weights"], atol=1e-6)
    assert arrs[(N.P_TOKEN_EMB, 0)].shape == (30, 8)


def test_input_validation_matches_reference_errors():
    import nimbleml_amd as nm

    m = nm.GPT(20, 8, 2, 1, 6)
    with pytest.raises(ValueError, match="exceeds maximum sequence length"):
        m.forward(np.zeros((1, 7), dtype=np.int64))
    with pytest.raises(ValueError, match="must be 2D"):
        m.forward(np.zeros((7,), dtype=np.int64))
    with pytest.raises(ValueError, match="out of range"):
        m.forward(np.full((1, 3), 20, dtype=np.int64))
    with pytest.raises(ValueError, match="label count"):
        m.compute_loss(np.zeros((1, 3), dtype=np.int64), np.zeros(4, dtype=np.int64))
    with pytest.raises(ValueError, match="exceeds maximum sequence length"):
        nm.generate(m, np.zeros((1, 4), dtype=np.int64), max_new_tokens=4)
    with pytest.raises(ValueError, match="divisible"):
        nm.GPT(20, 10, 3, 1, 6)
    with pytest.raises(ValueError, match="fused_trunk requires"):
        nm.GPT(20, 8, 2, 1, 6, fused_blocks=False, fused_trunk=True)
    with pytest.raises(ValueError, match="use_rope requires"):
        nm.GPT(20, 8, 2, 1, 6, fused_blocks=False, use_rope=True)
    m = nm.GPT(20, 8, 2, 2, 6, fused_blocks=False)  # models/gpt.py:66-67
    assert [type(b).__name__ for b in m.blocks.layers] == ["TransformerBlock"] * 2


def test_backend_device_and_dtype_selection():
    from nimbleml_amd import np_backend

    assert np_backend.device == "hip" and np_backend.using_gpu
    with pytest.raises(ValueError, match="HIP device only"):
        np_backend.set_device("cpu")
    assert np_backend.set_device("gpu") == "hip"
    old = np_backend.dtype
    try:
        assert np_backend.set_dtype("float16") == np.float16
        with pytest.raises(ValueError):
            np_backend.set_dtype("bfloat16")
    finally:
        np_backend.set_dtype(np.dtype(old).name)


def test_fused_trunk_names():
    import nimbleml_amd as nm

    m = nm.GPT(20, 8, 2, 2, 6, fused_trunk=True)
    names = [n for n, _ in nm.named_parameters(m)]
    assert "blocks.blocks.1.ffn.dense2.biases" in names and "blocks.ln.gamma" in names


def test_causal_mask_helpers():
    """utils/mask.py:8-27: triu(−inf, k=1) in the compute dtype, cached per (seq, dtype),
    no gradient; the modules take it for the causal kernels."""
    import nimbleml_amd as nm
    from nimbleml_amd.layers import _mask_mode

    old = nm.np_backend.dtype
    try:
        for dt in ("float32", "float16"):
            nm.set_dtype(dt)
            t = nm.causal_mask_tensor(5)
            a = nm.make_causal_mask(5)
            assert a.dtype == np.dtype(dt) and t.shape == (5, 5) and not t.requires_grad
            assert np.array_equal(a, np.triu(np.full((5, 5), -np.inf, dtype=dt), k=1))
            assert nm.causal_mask_tensor(5) is t
            assert _mask_mode(t, 5, np.dtype(dt), none_is_causal=False) == (1, None)
    finally:
        nm.set_dtype(np.dtype(old).name)
