"""GPU parity of each HIP kernel against the oracle / float64 closed forms.

Tolerances: integer work (gather, argmax, sampling choices) bit-exact; fp32 ops
≤ 1e-5 relative to float64 (GEMMs ≤ 1e-4); fp16 ops within one or two fp16 ulps of
the oracle's fp16 op-by-op result.
"""
import numpy as np
import pytest

from conftest import golden
from oracle import gpt_ref as R

pytestmark = pytest.mark.gpu


def _k():
    from nimbleml_amd import kernels

    return kernels


def _ulps16(a, b):
    a = np.asarray(a, np.float16).astype(np.float64)
    b = np.asarray(b, np.float16).astype(np.float64)
    scale = np.maximum(np.abs(b), 6.1e-5)
    return np.abs(a - b) / (scale * 2.0 ** -10)


@pytest.mark.parametrize("name", ["ops_fp32", "ops_fp16"])
def test_rmsnorm_matches_reference_fixture(gpu, name):
    f = golden(name)
    out = np.asarray(_k().fused_rmsnorm_forward(f["rms_x"], f["rms_g"])[0])
    if out.dtype == np.float16:
        assert _ulps16(out, f["rms_out"]).max() <= 2
    else:
        assert np.abs(out - f["rms_out"]).max() < 1e-5


@pytest.mark.parametrize("name", ["ops_fp32", "ops_fp16"])
def test_gelu_matches_reference_fixture(gpu, name):
    f = golden(name)
    out, tu = _k().fused_gelu_forward(f["gelu_x"])
    out = np.asarray(out)
    if out.dtype == np.float16:
        assert _ulps16(out, f["gelu_out"]).max() <= 1
    else:
        assert np.abs(out - f["gelu_out"]).max() < 2e-6
    x = f["gelu_x"].astype(np.float64)
    want_tu = np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3))
    assert np.abs(np.asarray(tu) - want_tu).max() < (2e-3 if out.dtype == np.float16 else 1e-6)


def test_gelu_fp16_every_input_bit_exact(gpu):
    """The fp16 GELU on every finite fp16 input equals the reference's NumPy float16
    evaluation (oracle gelu: each op rounded to fp16, kernels/fused_gelu.py:67-69) bit for
    bit — the standalone kernel (and its tanh output) and the GEMM epilogue (x·I + 0 with
    epilogue GELU, so the accumulator is the input exactly)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = bits.view(np.float16)
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore", invalid="ignore"):
        want = R.gelu(x)
        t = R.GELU_K * (x + R.GELU_COEF * x * x * x)
        want_tu = np.tanh(t)
    out, tu = _k().fused_gelu_forward(x)
    out, tu = np.asarray(out), np.asarray(tu)
    same = lambda a, b: (a == b) | (np.isnan(a) & np.isnan(b))
    bad = ~same(out, want)
    print(f"standalone: {int(bad.sum())} of {x.size} differ")
    assert not bad.any(), (x[bad][:8], out[bad][:8], want[bad][:8])
    assert np.all(same(tu, want_tu.astype(np.float32)))
    grid = x[: (x.size // 64) * 64].reshape(-1, 64)  # 992 × 64
    eye = np.eye(64, dtype=np.float16)
    got = np.asarray(_k().linear(grid, eye, np.zeros(64, np.float16), epilogue=2))
    bad = ~same(got, want[: grid.size].reshape(grid.shape))
    print(f"GEMM epilogue: {int(bad.sum())} of {grid.size} differ")
    assert not bad.any()
    # 4096 × 4096 outputs take the 256 × 256 tiles, whose GELU looks tanh up in a table:
    # every finite input (repeated to fill 4096 × 64) through x·[I | 0] + 0
    reps = -(-4096 * 64 // x.size)
    big = np.tile(x, reps)[: 4096 * 64].reshape(4096, 64)
    wbig = np.zeros((64, 4096), np.float16)
    wbig[:, :64] = eye
    got = np.asarray(_k().linear(big, wbig, np.zeros(4096, np.float16), epilogue=2))
    wbig_want = np.tile(want, reps)[: 4096 * 64].reshape(4096, 64)
    bad = ~same(got[:, :64], wbig_want)
    print(f"GEMM epilogue, 256 x 256 tiles: {int(bad.sum())} of {big.size} differ")
    assert not bad.any(), (big[bad][:8], got[:, :64][bad][:8], wbig_want[bad][:8])
    assert not got[:, 64:].any()


@pytest.mark.parametrize("name", ["ops_fp32", "ops_fp16"])
def test_embedding_gather_bit_exact(gpu, name):
    f = golden(name)
    out = np.asarray(_k().embedding_lookup(f["emb_w"], f["emb_ids"]))
    assert np.array_equal(out, f["emb_out"])


def test_embedding_with_positions_bit_exact(gpu):
    rng = np.random.default_rng(0)
    for dt in (np.float32, np.float16):
        E = rng.standard_normal((100, 48)).astype(dt)
        P = rng.standard_normal((20, 48)).astype(dt)
        ids = rng.integers(0, 100, (3, 17))
        out = np.asarray(_k().embedding_lookup(E, ids, pos_weights=P))
        assert np.array_equal(out, R.embed(E, P, ids))


@pytest.mark.parametrize("dt", [np.float32, np.float16])
@pytest.mark.parametrize("rows", [1, 3, 8, 9, 130, 300])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_linear_all_paths(gpu, dt, rows, epi):
    """GEMV (rows ≤ 8) and MFMA GEMM (rows > 8) with each epilogue, ragged tile edges."""
    rng = np.random.default_rng(rows * 10 + epi)
    k, n = 200, 136  # not multiples of the 128 tile
    x = rng.standard_normal((rows, k)).astype(dt)
    w = (rng.standard_normal((k, n)) * 0.1).astype(dt)
    b = rng.standard_normal(n).astype(dt)
    r = rng.standard_normal((rows, n)).astype(dt)
    out = np.asarray(_k().linear(x, w, b if epi else None, epilogue=epi,
                                 resid=r if epi == 3 else None)).astype(np.float64)
    acc = x.astype(np.float64) @ w.astype(np.float64)
    if dt == np.float16:
        acc = acc.astype(np.float16)
        lin = (acc + b).astype(np.float16) if epi else acc
        if epi == 2:
            lin = R.gelu(lin)
        if epi == 3:
            lin = (r + lin).astype(np.float16)
        tol = 3e-3 * max(1.0, np.abs(lin.astype(np.float64)).max())
        assert np.abs(out - lin.astype(np.float64)).max() <= tol
    else:
        lin = acc + b if epi else acc
        if epi == 2:
            lin = 0.5 * lin * (1 + np.tanh(np.sqrt(2 / np.pi) * (lin + 0.044715 * lin ** 3)))
        if epi == 3:
            lin = r + lin
        assert np.abs(out - lin).max() <= 1e-4 * max(1.0, np.abs(lin).max())


@pytest.mark.parametrize("shape", [(1, 4096, 1024), (2, 1024, 3072), (512, 1024, 1024),
                                   (700, 256, 4096)])
def test_linear_real_shapes_fp16(gpu, shape):
    rows, k, n = shape
    rng = np.random.default_rng(k)
    x = rng.standard_normal((rows, k)).astype(np.float16)
    w = (rng.standard_normal((k, n)) * 0.02).astype(np.float16)
    out = np.asarray(_k().linear(x, w)).astype(np.float64)
    want = (x.astype(np.float64) @ w.astype(np.float64)).astype(np.float16).astype(np.float64)
    assert np.abs(out - want).max() <= 2e-3 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("name", ["ops_fp32", "ops_fp16"])
def test_sdpa_matches_reference_fixture(gpu, name):
    f = golden(name)
    dk = f["sdpa_q"].shape[2]
    s = f["sdpa_q"].shape[1]
    out = np.asarray(_k().fused_sdpa_forward(f["sdpa_q"], f["sdpa_k"], f["sdpa_v"], float(dk) ** 0.5,
                                             R.causal_mask(s, f["sdpa_q"].dtype))[0])
    tol = 4e-3 if out.dtype == np.float16 else 1e-5
    assert np.abs(out.astype(np.float64) - f["sdpa_out"]).max() < tol


@pytest.mark.parametrize("dk", [8, 16, 32, 64, 128])
@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_sdpa_head_dims(gpu, dk, dt):
    rng = np.random.default_rng(dk)
    bh, s = 3, 150
    q, k, v = (rng.standard_normal((bh, s, dk)).astype(dt) for _ in range(3))
    out = np.asarray(_k().fused_sdpa_forward(q, k, v, float(dk) ** 0.5, R.causal_mask(s, dt))[0])
    want = R.sdpa(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                  float(dk) ** 0.5, R.causal_mask(s, np.float64))
    assert np.abs(out - want).max() < (6e-3 if dt == np.float16 else 1e-5)


@pytest.mark.parametrize("name", ["ops_fp32", "ops_fp16"])
def test_tied_ce_matches_reference_fixture(gpu, name):
    f = golden(name)
    loss = _k().fused_tied_crossentropy_forward(f["ce_h"], f["ce_e"], f["ce_y"])
    ref = float(f["ce_loss"])
    assert abs(loss - ref) <= (1e-3 if f["ce_h"].dtype == np.float16 else 1e-5) * abs(ref)


def test_tied_ce_ignore_index_and_closed_form(gpu):
    rng = np.random.default_rng(7)
    h = rng.standard_normal((300, 64)).astype(np.float32)
    e = (rng.standard_normal((1000, 64)) * 0.2).astype(np.float32)
    y = rng.integers(0, 1000, 300)
    y[::4] = -100
    loss = _k().fused_tied_crossentropy_forward(h, e, y, ignore_index=-100)
    keep = y != -100
    lg = h[keep].astype(np.float64) @ e.T.astype(np.float64)
    want = np.mean(np.log(np.exp(lg - lg.max(1, keepdims=True)).sum(1)) + lg.max(1)
                   - lg[np.arange(keep.sum()), y[keep]])
    assert abs(loss - want) < 1e-5 * abs(want)
    assert _k().fused_tied_crossentropy_forward(h, e, np.full(300, -100), ignore_index=-100) == 0.0


def _distinct_logits(rng, b, v, dt=np.float32):
    x = rng.standard_normal((b, v)) * 2
    return x.astype(dt)


def test_greedy_argmax_first_index_on_ties(gpu):
    rng = np.random.default_rng(1)
    lg = _distinct_logits(rng, 4, 32000, np.float16)
    lg[1, 100] = lg[1, 20000] = np.float16(50.0)  # tie: first index wins
    got = _k().sample_tokens(lg, temperature=0.0)
    assert np.array_equal(got, np.argmax(lg.astype(np.float32), axis=1))
    assert got[1] == 100


@pytest.mark.parametrize("top_k,top_p", [(0, 1.0), (50, 1.0), (1, 1.0), (0, 0.9), (40, 0.5),
                                         (0, 0.3)])
def test_sampling_matches_oracle(gpu, top_k, top_p):
    rng = np.random.default_rng(top_k * 7 + int(top_p * 10))
    for trial in range(3):
        lg = _distinct_logits(rng, 6, 4096)
        u = rng.random(6)
        got = _k().sample_tokens(lg, temperature=0.8, top_k=top_k, top_p=top_p, uniforms=u)
        want = [R.sample_logits(lg[b], temperature=0.8, top_k=top_k, top_p=top_p, u=u[b])
                for b in range(6)]
        assert list(got) == want, (trial, list(got), want)


@pytest.mark.parametrize("top_k,grid", [(30, True), (3000, False), (4096, False)])
def test_top_k_sampling_ties_and_large_k(gpu, top_k, grid):
    """Top-k without top-p: exact ties at the k-th largest logit (all tied elements are
    kept, generate.py:43-46), and k past the candidate buffer (2048) or equal to V (the
    device then takes the full-vocabulary scan)."""
    rng = np.random.default_rng(top_k + grid)
    b, v = 6, 4096
    if grid:
        lg = (rng.integers(-12, 12, (b, v)) * 0.25).astype(np.float32)
    else:
        lg = _distinct_logits(rng, b, v)
    u = rng.random(b)
    got = _k().sample_tokens(lg, temperature=0.8, top_k=top_k, top_p=1.0, uniforms=u)
    want = [R.sample_logits(lg[i], temperature=0.8, top_k=top_k, top_p=1.0, u=u[i])
            for i in range(b)]
    assert list(got) == want


@pytest.mark.parametrize("v", [32000, 32768, 4096, 520, 32776])
@pytest.mark.parametrize("top_k", [1, 50, 256, 257])
def test_top_k_sampling_fp16_rows(gpu, v, top_k):
    """fp16 logits, top-k without top-p: the register-resident draw (1 <= k <= 256, V a
    multiple of 8 up to 32768) and, past those bounds or when more than 512 elements
    reach its lower bound, the general path give the oracle's token, for random rows,
    rows with exact ties at the k-th largest value, an ascending row and a constant row."""
    rng = np.random.default_rng(v + top_k)
    b = 8
    lg = (rng.standard_normal((b, v)) * 2).astype(np.float16)
    lg[1] = (rng.integers(-8, 8, v) * 0.5).astype(np.float16)
    lg[2] = np.linspace(-4, 4, v).astype(np.float16)
    lg[3] = np.float16(0.0)
    u = rng.random(b)
    got = _k().sample_tokens(lg, temperature=0.8, top_k=top_k, top_p=1.0, uniforms=u)
    want = [R.sample_logits(lg[i], temperature=0.8, top_k=top_k, top_p=1.0, u=u[i])
            for i in range(b)]
    assert list(got) == want


def test_top_k_sampling_fp16_with_repetition_penalty(gpu):
    rng = np.random.default_rng(13)
    b, v = 6, 32000
    lg = (rng.standard_normal((b, v)) * 2).astype(np.float16)
    top = np.argsort(-lg.astype(np.float32), axis=1)
    hist = [list(top[i, :40:3]) + [int(t) for t in rng.integers(0, v, 50)] for i in range(b)]
    u = rng.random(b)
    got = _k().sample_tokens(lg, temperature=0.7, top_k=50, uniforms=u, history=hist,
                             repetition_penalty=1.3)
    want = [R.sample_logits(lg[i], temperature=0.7, top_k=50, top_p=1.0, u=u[i],
                            token_ids=hist[i], repetition_penalty=1.3) for i in range(b)]
    assert list(got) == want


def test_sampling_with_repetition_penalty(gpu):
    rng = np.random.default_rng(11)
    lg = _distinct_logits(rng, 3, 1000)
    hist = [[1, 5, 5, 9], [int(np.argmax(lg[1]))], list(range(0, 1000, 7))]
    u = rng.random(3)
    for temp, k in ((0.0, 0), (0.7, 20)):
        got = _k().sample_tokens(lg, temperature=temp, top_k=k, uniforms=u, history=hist,
                                 repetition_penalty=1.7)
        want = [R.sample_logits(lg[b], temperature=temp, top_k=k, top_p=1.0, u=u[b],
                                token_ids=hist[b], repetition_penalty=1.7) for b in range(3)]
        assert list(got) == want


@pytest.mark.parametrize("top_k", [0, 30])
def test_top_p_exact_ties_descending_index(gpu, top_k):
    """Equal probabilities in the top-p walk come in descending index order — the
    order argsort(probs)[::-1] gives when the ascending sort is stable
    (models/generate.py:50). Logits on a coarse grid make many exact ties."""
    rng = np.random.default_rng(42 + top_k)
    b, v = 8, 512
    lg = (rng.integers(-12, 12, (b, v)) * 0.25).astype(np.float32)
    u = rng.random(b)

    def stable_pick(row, uu):
        x = row / np.float32(0.8)
        if top_k:
            th = np.partition(x, -top_k)[-top_k]
            x = np.where(x < th, np.float32(-1e9), x)
        p = np.exp(x - x.max())
        p = p / p.sum()
        order = np.argsort(p, kind="stable")[::-1]
        sp = p[order]
        cdf = np.cumsum(sp)
        mask = cdf > 0.9
        mask[0] = False
        sp = np.where(mask, 0.0, sp)
        sp = sp / sp.sum()
        return int(order[R.choice_from_uniform(sp, uu)])

    got = _k().sample_tokens(lg, temperature=0.8, top_k=top_k, top_p=0.9, uniforms=u)
    assert list(got) == [stable_pick(lg[i], u[i]) for i in range(b)]


@pytest.mark.parametrize("rows", [9, 17, 32, 33, 64])
@pytest.mark.parametrize("k", [128, 1024, 4096])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_linear_skinny_fp16(gpu, rows, k, epi):
    """Batched-decode shapes (8 < rows ≤ 64, K a multiple of 128): the skinny MFMA GEMM."""
    rng = np.random.default_rng(rows * 100 + k + epi)
    n = 200  # ragged against the 16-column tile
    x = rng.standard_normal((rows, k)).astype(np.float16)
    w = (rng.standard_normal((k, n)) * (1.0 / np.sqrt(k))).astype(np.float16)
    b = rng.standard_normal(n).astype(np.float16)
    r = rng.standard_normal((rows, n)).astype(np.float16)
    out = np.asarray(_k().linear(x, w, b if epi else None, epilogue=epi,
                                 resid=r if epi == 3 else None)).astype(np.float64)
    acc = (x.astype(np.float64) @ w.astype(np.float64)).astype(np.float16)
    lin = (acc + b).astype(np.float16) if epi else acc
    if epi == 2:
        lin = R.gelu(lin)
    if epi == 3:
        lin = (r + lin).astype(np.float16)
    want = lin.astype(np.float64)
    # acc may differ by one fp16 ulp (an fp32 sum in another order, rounded once); each
    # later rounding adds one ulp of its own operands, so the bound scales with the
    # operand magnitudes, not with a result that may cancel to ~0.
    scale = np.abs(acc.astype(np.float64))
    if epi:
        scale = scale + np.abs(b.astype(np.float64))
    if epi == 3:
        scale = scale + np.abs(r.astype(np.float64))
    tol = 2.0 * 2.0 ** -10 * (scale + np.abs(want)) + 1e-4
    assert np.all(np.abs(out - want) <= tol), float(np.max(np.abs(out - want) / tol))


@pytest.mark.parametrize("rows,k,n", [(9, 2048, 8200), (32, 1024, 32000), (64, 512, 8198),
                                      (33, 1024, 8192), (17, 1536, 12345)])
def test_linear_skinny_wide_fp16(gpu, rows, k, n):
    """Head-like shapes (8 < rows <= 64, N >= 8192, no epilogue, K a multiple of 512):
    x staged once per workgroup, each wave streaming 16 W rows over the whole K; ragged
    N against the 64-row workgroup and the 4-column stores. K = 1536 (not a multiple of
    512) and 33 rows at K = 1024 (x too large for two workgroups' LDS) take the skinny
    kernel: both give x·Wᵀ within the fp16 bound."""
    rng = np.random.default_rng(rows * 1000 + n)
    x = rng.standard_normal((rows, k)).astype(np.float16)
    w = (rng.standard_normal((k, n)) * (1.0 / np.sqrt(k))).astype(np.float16)
    out = np.asarray(_k().linear(x, w, None, epilogue=0)).astype(np.float64)
    acc = (x.astype(np.float64) @ w.astype(np.float64))
    want = acc.astype(np.float16).astype(np.float64)
    tol = 2.0 * 2.0 ** -10 * (np.abs(acc) + np.abs(want)) + 1e-4
    assert np.all(np.abs(out - want) <= tol), float(np.max(np.abs(out - want) / tol))


@pytest.mark.parametrize("rows,k,n,epi", [(4096, 256, 4096, 0), (4096, 192, 4224, 1),
                                          (4096, 128, 4224, 2), (3000, 256, 4224, 3),
                                          (4096, 128, 4099, 3), (4096, 64, 4097, 2),
                                          (1024, 192, 3072, 1), (700, 256, 1000, 3),
                                          (300, 128, 520, 2), (515, 64, 136, 0),
                                          (700, 64, 1001, 3), (600, 128, 1030, 1),
                                          (17317, 128, 1024, 3), (17317, 64, 3072, 1)])
def test_linear_big_tile_fp16(gpu, rows, k, n, epi):
    """Prefill-sized shapes on the direct-to-LDS MFMA GEMM: 256×256 tiles where there are
    ≥ 256 of them, 128×128 tiles below that (rows ≤ 1024) and where the last round of big
    tiles would be short (17317 × 1024: 272 big tiles; 17317 × 3072, 816, stays on the
    big ones), with ragged last column tiles
    (n = 4224, 1000, 520, 136), ragged last row tiles (rows = 3000, 700, 300, 515), and
    widths that are not multiples of 4 (4099, 4097, 1001, 1030: the epilogue's
    element-by-element path instead of 8-byte runs)."""
    rng = np.random.default_rng(rows + k + n + epi)
    x = rng.standard_normal((rows, k)).astype(np.float16)
    w = (rng.standard_normal((k, n)) * (1.0 / np.sqrt(k))).astype(np.float16)
    b = rng.standard_normal(n).astype(np.float16)
    r = rng.standard_normal((rows, n)).astype(np.float16)
    out = np.asarray(_k().linear(x, w, b if epi else None, epilogue=epi,
                                 resid=r if epi == 3 else None)).astype(np.float64)
    acc = (x.astype(np.float64) @ w.astype(np.float64)).astype(np.float16)
    lin = (acc + b).astype(np.float16) if epi else acc
    if epi == 2:
        lin = R.gelu(lin)
    if epi == 3:
        lin = (r + lin).astype(np.float16)
    want = lin.astype(np.float64)
    scale = np.abs(acc.astype(np.float64))
    if epi:
        scale = scale + np.abs(b.astype(np.float64))
    if epi == 3:
        scale = scale + np.abs(r.astype(np.float64))
    tol = 2.0 * 2.0 ** -10 * (scale + np.abs(want)) + 1e-4
    assert np.all(np.abs(out - want) <= tol), float(np.max(np.abs(out - want) / tol))


@pytest.mark.parametrize("dk", [64, 128])
def test_sdpa_mfma_long_fp16(gpu, dk):
    """The matrix-core flash kernel over many 64-key tiles and a ragged last query tile."""
    rng = np.random.default_rng(dk + 1)
    bh, s = 2, 1000
    q, k, v = (rng.standard_normal((bh, s, dk)).astype(np.float16) for _ in range(3))
    out = np.asarray(_k().fused_sdpa_forward(q, k, v, float(dk) ** 0.5,
                                             R.causal_mask(s, np.float16))[0]).astype(np.float64)
    want = R.sdpa(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                  float(dk) ** 0.5, R.causal_mask(s, np.float64))
    assert np.abs(out - want).max() < 6e-3


@pytest.mark.parametrize("dk", [64, 128])
@pytest.mark.parametrize("s", [1, 2, 63, 64, 65, 127, 129, 192, 257])
def test_sdpa_mfma_tile_edges_fp16(gpu, dk, s):
    """The fp16 matrix-core kernels at lengths around the 64-key tile and the 128-query
    workgroup: one, two and three key tiles, partial last tiles, waves past the end."""
    rng = np.random.default_rng(dk * 1000 + s)
    bh = 3
    q, k, v = (rng.standard_normal((bh, s, dk)).astype(np.float16) for _ in range(3))
    out = np.asarray(_k().fused_sdpa_forward(q, k, v, float(dk) ** 0.5,
                                             R.causal_mask(s, np.float16))[0]).astype(np.float64)
    want = R.sdpa(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                  float(dk) ** 0.5, R.causal_mask(s, np.float64))
    assert np.abs(out - want).max() < 6e-3


@pytest.mark.parametrize("dk", [16, 40, 64, 96, 128, 256])
@pytest.mark.parametrize("seq", [1, 37, 200])
def test_flash_sdpa_forward_device_reference_arguments(gpu, dk, seq):
    """flash_sdpa_forward_device with the reference's arguments (module.cpp:231-242):
    `scale` = 1/sqrt(dk) multiplies the scores; out, m and l against the float64
    restatement of sdpa_cuda.cu:40-77."""
    from oracle import grad_ref as G

    rng = np.random.default_rng(dk + seq)
    q, k, v = (rng.standard_normal((3, seq, dk)).astype(np.float32) for _ in range(3))
    out, m, lsum = _k().flash_sdpa_forward(q, k, v, np.sqrt(dk))
    want, wm, wl = G.flash_forward(q.astype(np.float64), k.astype(np.float64),
                                   v.astype(np.float64), 1.0 / np.sqrt(dk))
    assert np.abs(np.asarray(out) - want).max() < 1e-5
    assert np.abs(np.asarray(m) - wm).max() < 1e-5 * max(1.0, np.abs(wm).max())
    assert (np.abs(np.asarray(lsum) - wl) / wl).max() < 1e-5


@pytest.mark.parametrize("dk", [16, 40, 64, 96, 128, 256])
def test_flash_sdpa_backward_device(gpu, dk):
    """flash_sdpa_backward_device (module.cpp:243-257): gradients against the float64
    restatement of sdpa_cuda.cu:79-133, with the forward's m and l."""
    from oracle import grad_ref as G

    rng = np.random.default_rng(dk)
    seq = 150
    q, k, v, go = (rng.standard_normal((2, seq, dk)).astype(np.float32) for _ in range(4))
    _, m, lsum = _k().flash_sdpa_forward(q, k, v, np.sqrt(dk))
    grads = _k().flash_sdpa_backward(go, q, k, v, m, lsum, np.sqrt(dk))
    want = G.flash_backward(*(a.astype(np.float64) for a in (go, q, k, v)), 1.0 / np.sqrt(dk))
    for got, w in zip(grads, want):
        assert np.abs(np.asarray(got) - w).max() <= 2e-5 * np.abs(w).max()


@pytest.mark.parametrize("rows,dim", [(1, 64), (37, 96), (300, 1024)])
def test_rmsnorm_backward_device(gpu, rows, dim):
    """rmsnorm_backward_device (module.cpp:271-284): grad_x and grad_gamma (overwritten)
    against the float64 restatement."""
    from oracle import grad_ref as G

    rng = np.random.default_rng(rows)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    go = rng.standard_normal((rows, dim)).astype(np.float32)
    gx, gg = _k().fused_rmsnorm_backward(go, x, g)
    wx, wg = G.rmsnorm_backward(go.astype(np.float64), x.astype(np.float64), g.astype(np.float64))
    assert np.abs(np.asarray(gx) - wx).max() <= 1e-5 * np.abs(wx).max()
    assert np.abs(np.asarray(gg) - wg).max() <= 1e-5 * np.abs(wg).max()
    gx2, gg2 = _k().fused_rmsnorm_backward(go, x, g)  # grad_gamma overwritten, not added
    assert np.array_equal(np.asarray(gg2), np.asarray(gg))
