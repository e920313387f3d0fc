"""GPU parity of the tied lm_head + fused greedy argmax, the fused MLP block and
the RMSNorm kernels against the CPU oracle.

Bars: argmax token ids identical to the oracle (lowest index on exact ties);
fused MLP BF16 <= 1e-2 vs FP64, INT8 <= 1e-3 vs dequant-then-matmul, FP32
<= 1e-5 vs FP64; RMSNorm <= 1e-6 normwise vs FP64 (FP32 in/out).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


# ----------------------------------------------------------------------------
# lm_head + argmax
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("M", [1, 5, 32, 37, 100])
def test_lmhead_argmax_bf16(qw, ctx, oracle, M):
    V, K = 20000, 1024
    E = oracle.normal((V, K), 301, 0.0, 0.02)
    h = oracle.normal((M, K), 302 + M)
    Eb = oracle.to_bf16(E)
    hb = oracle.to_bf16(h)
    w = qw.Weight.pack(ctx, Eb, qw.WFMT_BF16, src_code=qw.BF16)
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    mx = torch.empty(M, device="cuda")
    qw.lmhead_argmax(ctx, w, dev(oracle.from_bf16(hb), torch.bfloat16), ids, mx)
    torch.cuda.synchronize()
    ref_ids, ref_max = oracle.lmhead_argmax_bf16(Eb, hb)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    np.testing.assert_allclose(mx.cpu().numpy(), ref_max, rtol=1e-4, atol=1e-5)
    # repeat: keys and counters must have been returned to zero
    ids2 = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    qw.lmhead_argmax(ctx, w, dev(oracle.from_bf16(hb), torch.bfloat16), ids2)
    torch.cuda.synchronize()
    assert np.array_equal(ids2.cpu().numpy(), ref_ids)


@pytest.mark.parametrize("M", [1, 8, 70])
def test_lmhead_argmax_int8(qw, ctx, oracle, M):
    V, K = 12000, 1024
    E = oracle.normal((V, K), 311, 0.0, 0.02)
    h = oracle.normal((M, K), 312)
    w = qw.Weight.pack(ctx, E, qw.WFMT_INT8)
    q, s = w.unpack()
    hs = host(dev(h, torch.float16))
    ids = torch.empty(M, dtype=torch.int32, device="cuda")
    qw.lmhead_argmax(ctx, w, dev(h, torch.float16), ids)
    torch.cuda.synchronize()
    ref_ids, _ = oracle.lmhead_argmax_int8(q, s, hs)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)


def test_lmhead_argmax_ties_lowest_index(qw, ctx, oracle):
    """Planted exact ties: rows 3, 700 and 9000 identical and maximal for
    token 0 -> 3; a planted unique maximum at 12345 for token 1."""
    V, K = 16000, 128
    E = np.round(oracle.normal((V, K), 321, 0.0, 0.02) * 256) / 256
    h = np.zeros((2, K), np.float32)
    h[0, :] = 1.0 / 64
    h[1, :] = -1.0 / 64
    big = np.full(K, 0.5, np.float32)
    for r in (3, 700, 9000):
        E[r] = big
    E[12345] = -big
    w = qw.Weight.pack(ctx, E, qw.WFMT_F32)
    ids = torch.empty(2, dtype=torch.int32, device="cuda")
    qw.lmhead_argmax(ctx, w, dev(h), ids)
    torch.cuda.synchronize()
    got = ids.cpu().numpy()
    ref, _ = oracle.lmhead_argmax(E, h)
    assert got[0] == 3 and got[1] == 12345
    assert np.array_equal(got, ref)


# ----------------------------------------------------------------------------
# fused MLP block
# ----------------------------------------------------------------------------

def _mlp_weights(oracle, H, I, seed):
    G = oracle.normal((I, H), seed, 0.0, 0.02)
    U = oracle.normal((I, H), seed + 1, 0.0, 0.02)
    D = oracle.normal((H, I), seed + 2, 0.0, 0.02)
    return G, U, D


@pytest.mark.parametrize("M", [1, 8, 32, 128])
def test_mlp_fused_bf16(qw, ctx, oracle, relerr, M):
    H, I = 1024, 3584
    G, U, D = _mlp_weights(oracle, H, I, 401)
    gamma = oracle.normal((H,), 404, 0.0, 0.02)
    x = oracle.normal((M, H), 405)
    gu = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16)
    dn = qw.Weight.pack(ctx, D, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    y = torch.empty(M, H, device="cuda")
    qw.mlp_fused(ctx, gu, dn, xt, y, gamma=dev(gamma), residual=xt)
    torch.cuda.synchronize()
    xs = host(xt)
    ref = oracle.mlp_block_f64(G, U, D, gamma, xs)
    assert relerr(host(y), ref) <= 1e-2
    # against the bf16-rounded weights the error is far smaller
    ref_b = oracle.mlp_block_f64(oracle.round_bf16(G), oracle.round_bf16(U), oracle.round_bf16(D), gamma, xs)
    assert relerr(host(y), ref_b) <= 2e-3
    assert ctx.device_error() == 0


def test_mlp_fused_repeat_in_place(qw, ctx, oracle, relerr):
    """Repeated launches must give identical results (device counters of the
    one-launch path return to zero; split-K partials are summed in a fixed
    order), and the in-place form (y aliases x and the residual) must match
    the out-of-place one."""
    H, I, M = 1024, 3584, 1
    G, U, D = _mlp_weights(oracle, H, I, 431)
    gamma = oracle.normal((H,), 434, 0.0, 0.02)
    gu = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16)
    dn = qw.Weight.pack(ctx, D, qw.WFMT_BF16)
    x0 = oracle.normal((M, H), 435)
    xt = dev(x0)
    g = dev(gamma)
    ys = torch.empty(50, M, H, device="cuda")
    for i in range(50):
        qw.mlp_fused(ctx, gu, dn, xt, ys[i], gamma=g, residual=xt)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    got = ys.cpu().numpy()
    assert (got == got[0][None]).all()
    ref = oracle.mlp_block_f64(oracle.round_bf16(G), oracle.round_bf16(U), oracle.round_bf16(D), gamma, x0)
    assert relerr(got[0], ref) <= 2e-3
    qw.mlp_fused(ctx, gu, dn, xt, xt, gamma=g, residual=xt)       # in place
    torch.cuda.synchronize()
    assert np.array_equal(host(xt), got[0])


@pytest.mark.parametrize("M", [1, 32, 128])
def test_mlp_fused_int8(qw, ctx, oracle, relerr, M):
    H, I = 1024, 3584
    G, U, D = _mlp_weights(oracle, H, I, 411)
    x = oracle.normal((M, H), 415)
    gu = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_INT8)
    dn = qw.Weight.pack(ctx, D, qw.WFMT_INT8)
    xt = dev(x, torch.float16)
    y = torch.empty(M, H, device="cuda")
    qw.mlp_fused(ctx, gu, dn, xt, y)
    torch.cuda.synchronize()
    qgu, sgu = gu.unpack()
    qd, sd = dn.unpack()
    # reference: dequant-then-matmul MLP (FP32 weights q*s)
    Gd = qgu[:I].astype(np.float32) * sgu[:I, None]
    Ud = qgu[I:].astype(np.float32) * sgu[I:, None]
    Dd = qd.astype(np.float32) * sd[:, None]
    ref = oracle.mlp(Gd, Ud, Dd, host(xt))
    assert relerr(host(y), ref) <= 1e-3


def test_mlp_fused_f32_matches_reference_mlp(qw, ctx, oracle, relerr):
    """FP32 weights: config-1 precision, against MLP::forward restated."""
    H, I, M = 1024, 3584, 2
    G, U, D = _mlp_weights(oracle, H, I, 421)
    x = oracle.normal((M, H), 425)
    gu = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_F32)
    dn = qw.Weight.pack(ctx, D, qw.WFMT_F32)
    y = torch.empty(M, H, device="cuda")
    qw.mlp_fused(ctx, gu, dn, dev(x), y)
    torch.cuda.synchronize()
    assert relerr(host(y), oracle.mlp_f64(G, U, D, x)) <= 1e-5
    assert relerr(host(y), oracle.mlp(G, U, D, x)) <= 1e-5


# ----------------------------------------------------------------------------
# RMSNorm
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("M,K", [(1, 1024), (7, 1024), (3, 2048), (2, 100)])
def test_rmsnorm(qw, ctx, oracle, relerr, M, K):
    x = oracle.normal((M, K), 501) * 2.0
    w = oracle.normal((K,), 502, 0.0, 0.02)
    y = torch.empty(M, K, device="cuda")
    qw.rmsnorm(ctx, dev(x), dev(w), y)
    torch.cuda.synchronize()
    assert relerr(host(y), oracle.rmsnorm_f64(x, w)) <= 1e-6


def test_rmsnorm_constant_closed_form(qw, ctx, oracle):
    """x = c everywhere: y = c / sqrt(c^2 + eps) * (1 + w)."""
    K, c = 1024, 0.75
    x = np.full((1, K), c, np.float32)
    w = oracle.normal((K,), 503, 0.0, 0.02)
    y = torch.empty(1, K, device="cuda")
    qw.rmsnorm(ctx, dev(x), dev(w), y)
    torch.cuda.synchronize()
    ref = c / np.sqrt(c * c + 1e-6) * (1.0 + w.astype(np.float64))
    np.testing.assert_allclose(host(y)[0], ref, rtol=2e-6)


@pytest.mark.parametrize("M", [1, 16])
def test_residual_rmsnorm(qw, ctx, oracle, relerr, M):
    K = 1024
    r = oracle.normal((M, K), 511)
    a = oracle.normal((M, K), 512)
    w = oracle.normal((K,), 513, 0.0, 0.02)
    rt = dev(r)
    normed = torch.empty(M, K, device="cuda")
    qw.residual_rmsnorm(ctx, rt, dev(a), rt, normed, dev(w))      # in place residual
    torch.cuda.synchronize()
    ro, no = oracle.residual_rmsnorm(r, a, w)
    assert np.array_equal(host(rt), ro)                            # the add is exact fp32
    assert relerr(host(normed), oracle.rmsnorm_f64(ro, w)) <= 1e-6


def test_silu_mul(qw, ctx, oracle, relerr):
    n = 3584 * 3
    g = oracle.normal((n,), 521) * 3
    u = oracle.normal((n,), 522)
    h = torch.empty(n, device="cuda")
    qw.silu_mul(ctx, dev(g), dev(u), h)
    torch.cuda.synchronize()
    gd = g.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * u
    assert relerr(host(h), ref) <= 1e-6


@pytest.mark.parametrize("fmt,M", [("bf16", 1), ("bf16", 8), ("int8", 1), ("int8", 16), ("f32", 2),
                                   ("bf16x32", 1), ("bf16x32", 4), ("int8x32", 3)])
def test_mlp_one_launch_path(qw, oracle, relerr, fmt, M):
    """The single-launch MLP kernel (the decode default; QW_MLP_FUSED=1 set
    explicitly) against the oracle, repeated to check its counters reset.
    bf16x32 / int8x32: FP32 activations (staged through LDS as hi + lo),
    the engine's residual stream; f32: FP32 weights (two-launch path)."""
    import os
    os.environ["QW_MLP_FUSED"] = "1"
    try:
        c = qw.Context(0)
    finally:
        del os.environ["QW_MLP_FUSED"]
    H, I = 1024, 3584
    f = {"bf16": qw.WFMT_BF16, "int8": qw.WFMT_INT8, "f32": qw.WFMT_F32,
         "bf16x32": qw.WFMT_BF16, "int8x32": qw.WFMT_INT8}[fmt]
    xdt = {"bf16": torch.bfloat16, "int8": torch.float16, "f32": torch.float32,
           "bf16x32": torch.float32, "int8x32": torch.float32}[fmt]
    G, U, D = _mlp_weights(oracle, H, I, 441)
    gamma = oracle.normal((H,), 444, 0.0, 0.02)
    x = oracle.normal((M, H), 445)
    gu = qw.Weight.pack_glu(c, G, U, f)
    dn = qw.Weight.pack(c, D, f)
    xt = dev(x, xdt)
    ys = [torch.empty(M, H, device="cuda") for _ in range(3)]
    for y in ys:
        qw.mlp_fused(c, gu, dn, xt, y, gamma=dev(gamma), residual=xt)
    torch.cuda.synchronize()
    assert c.device_error() == 0
    assert all(torch.equal(ys[0], y) for y in ys[1:])
    xs = host(xt)
    if fmt in ("int8", "int8x32"):
        qgu, sgu = gu.unpack()
        qd, sd = dn.unpack()
        Gd = qgu[:I].astype(np.float32) * sgu[:I, None]
        Ud = qgu[I:].astype(np.float32) * sgu[I:, None]
        Dd = qd.astype(np.float32) * sd[:, None]
        ref = oracle.mlp_block(Gd, Ud, Dd, gamma, xs)
        bar = 1e-3
    elif fmt in ("bf16", "bf16x32"):
        ref = oracle.mlp_block_f64(G, U, D, gamma, xs)
        bar = 1e-2
    else:
        ref = oracle.mlp_block_f64(G, U, D, gamma, xs)
        bar = 1e-5
    assert relerr(host(ys[0]), ref) <= bar
    del gu, dn
    c.close()


@pytest.mark.gpu
@pytest.mark.parametrize("M,V,dt", [(1, 248320, "f32"), (3, 5000, "f32"), (130, 4099, "bf16"), (1, 7, "f32")])
def test_argmax_rows(qw, ctx, oracle, M, V, dt):
    """Row argmax over materialized logits against the reference Sampler rule
    (oracle argmax_first), with planted exact ties in every other row."""
    L = oracle.normal((M, V), 600 + M)
    for m in range(0, M, 2):
        L[m, [V // 3, V - 1, V // 2]] = 7.5
    if dt == "bf16":
        L = oracle.round_bf16(L)
    t = dev(L).to(torch.bfloat16 if dt == "bf16" else torch.float32)
    ids = torch.empty(M, dtype=torch.int32, device="cuda")
    mx = torch.empty(M, device="cuda")
    for _ in range(2):  # second call checks the keys/counter were reset
        qw.argmax_rows(ctx, t, ids, mx)
        torch.cuda.synchronize()
        ref = [oracle.argmax_first(r) for r in L]
        assert list(ids.cpu().numpy()) == ref
        assert np.array_equal(mx.cpu().numpy(), L.max(axis=1))
