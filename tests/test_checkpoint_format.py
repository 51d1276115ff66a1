"""Training-checkpoint format on the host (no GPU): the reference's layout
(utils/saveload.py:303-358) — ``model/<name>`` arrays plus the JSON ``_checkpoint_meta`` —
and its errors. The optimizer-state round trip runs on the GPU (test_gpu_checkpoint.py)."""
import json

import numpy as np
import pytest

from oracle.weights import GPTConfig, make_weights

CFG = GPTConfig(128, 32, 2, 2, 16)


def _model(seed):
    import nimbleml_amd as nm

    m = nm.GPT(CFG.vocab_size, CFG.d_model, CFG.num_heads, CFG.num_layers, CFG.max_seq_len)
    nm.load_arrays(m, make_weights(CFG, seed=seed, dtype=np.float32, rich=True))
    return m


def test_checkpoint_layout_and_round_trip(tmp_path):
    import nimbleml_amd as nm
    from nimbleml_amd.saveload import named_parameters

    a = _model(1)
    path = str(tmp_path / "ck.npz")
    nm.save_checkpoint(path, a, step=7, extra={"epoch": 2})
    with np.load(path) as data:
        meta = json.loads(str(data["_checkpoint_meta"]))
        assert meta == {"version": 1, "step": 7, "extra": {"epoch": 2}}
        names = {k for k in data.files if k != "_checkpoint_meta"}
    assert names == {f"model/{n}" for n, _ in named_parameters(a)}
    b = _model(2)
    assert nm.load_checkpoint(path, b) == {"step": 7, "extra": {"epoch": 2}}
    for (n, p), (_, q) in zip(named_parameters(a), named_parameters(b)):
        assert np.array_equal(np.asarray(p.data), np.asarray(q.data)), n


def test_checkpoint_errors(tmp_path):
    import nimbleml_amd as nm

    a = _model(1)
    ck, w = str(tmp_path / "ck.npz"), str(tmp_path / "w.npz")
    nm.save_checkpoint(ck, a)
    nm.save(a, w)
    with pytest.raises(ValueError, match="training checkpoint"):
        nm.load(a, ck)
    with pytest.raises(ValueError, match="Not a training checkpoint"):
        nm.load_checkpoint(w, a)
    opt = nm.AdamW(a.parameters())
    with pytest.raises(ValueError, match="does not contain optimizer state"):
        nm.load_checkpoint(ck, a, opt)
    with pytest.raises(TypeError):
        nm.AdamW([object()])
