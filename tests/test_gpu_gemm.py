"""GPU parity of the MFMA GEMM path (M >= 33 tokens, BF16 weights and
activations) against the CPU oracle.

Bars: <= 2e-5 normwise vs FP64 on the exact stored operands for FP32 outputs
(one wrong k, row or token shows up as an O(1) error); BF16 outputs carry
one rounding (<= 4e-3); argmax ids identical to the oracle.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", params=["128x4", "256x4", "256x8", "r64", "da"])
def ctx(qw, request):
    """A context that takes the GEMM for every BF16 / INT8 call from 33 tokens
    on (the default routing sends small-N shapes to the chunked small-M
    kernels), with each block shape: 256 rows x 128 tokens x 4 waves, 256 x
    256 x 4, 256 x 256 x 8 (INT8 weights always run 8 waves on 256-row
    blocks), 64 rows x 128 tokens x 4 waves ("r64"), and the direct-A kernel
    (qw_gemm_da.hip) on every BF16 x BF16 call it can take ("da"; INT8,
    argmax and shapes it does not take run the 256-row GEMM)."""
    import os
    if request.param == "r64":
        env = {"QW_GEMM_MIN_M": "33", "QW_GEMM_ROWS": "64"}
    elif request.param == "da":
        env = {"QW_GEMM_MIN_M": "33", "QW_GEMM_ROWS": "256", "QW_GEMM_DA": "2"}
    else:
        tile, waves = request.param.split("x")
        env = {"QW_GEMM_MIN_M": "33", "QW_GEMM_TILE_M": tile, "QW_GEMM_WAVES": waves, "QW_GEMM_ROWS": "256"}
    os.environ.update(env)
    try:
        c = qw.Context(0)
    finally:
        for k in env:
            del os.environ[k]
    yield c
    torch.cuda.synchronize()
    c.close()


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("M,N,K", [(33, 40, 64), (64, 1024, 1024), (256, 256, 128), (300, 1024, 3584),
                                   (1000, 2048, 1024), (517, 16, 1024), (256, 8224, 1024)])
def test_gemm_parity(qw, ctx, oracle, relerr, M, N, K):
    W = oracle.normal((N, K), 700 + N, 0.0, 0.02)
    x = oracle.normal((M, K), 701 + M)
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    y = torch.empty(M, N, device="cuda")
    qw.linear(ctx, w, xt, y)
    torch.cuda.synchronize()
    ref = oracle.linear_f64(oracle.round_bf16(W), host(xt))
    assert relerr(host(y), ref) <= 2e-5
    assert relerr(host(y), oracle.linear_f64(W, host(xt))) <= 1e-2


def test_gemm_onehot_tokens_and_rows(qw, ctx, oracle):
    """Token j = e_{k(j)} picks column k(j) of W: catches token/row swaps."""
    M, N, K = 96, 512, 256
    W = np.round(oracle.normal((N, K), 710, 0.0, 0.02) * 1024) / 1024
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    ks = (np.arange(M) * 37) % K
    x = np.zeros((M, K), np.float32)
    x[np.arange(M), ks] = 1.0
    y = torch.empty(M, N, device="cuda")
    qw.linear(ctx, w, dev(x, torch.bfloat16), y)
    torch.cuda.synchronize()
    Wb = oracle.round_bf16(W)
    assert np.array_equal(host(y), Wb[:, ks].T)


@pytest.mark.parametrize("M", [64, 300])
def test_gemm_glu(qw, ctx, oracle, relerr, M):
    I, H = 3584, 1024
    G = oracle.normal((I, H), 720, 0.0, 0.02)
    U = oracle.normal((I, H), 721, 0.0, 0.02)
    x = oracle.normal((M, H), 722)
    w = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    h = torch.empty(M, I, device="cuda")
    qw.linear(ctx, w, xt, h)
    torch.cuda.synchronize()
    xs = host(xt).astype(np.float64)
    g = xs @ oracle.round_bf16(G).astype(np.float64).T
    u = xs @ oracle.round_bf16(U).astype(np.float64).T
    ref = g / (1.0 + np.exp(-g)) * u
    assert relerr(host(h), ref) <= 1e-4


@pytest.mark.parametrize("ydt", ["bf16", "f32"])
def test_gemm_residual_norm_split(qw, ctx, oracle, relerr, ydt):
    """RMSNorm prologue (through the workspace), residual epilogue, and the
    full-attention Q/gate split, all on the GEMM path."""
    M, K = 130, 1024
    heads, D = 8, 256
    N = 2 * heads * D
    W = oracle.normal((N, K), 730, 0.0, 0.02)
    gamma = oracle.normal((K,), 731, 0.0, 0.02)
    x = oracle.normal((M, K), 732) * 2.0
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    ydtype = torch.bfloat16 if ydt == "bf16" else torch.float32
    q = torch.empty(M, heads * D, device="cuda", dtype=ydtype)
    g = torch.empty(M, heads * D, device="cuda", dtype=ydtype)
    qw.linear(ctx, w, xt, q, y2=g, split_period=D, gamma=dev(gamma))
    torch.cuda.synchronize()
    xn = oracle.rmsnorm_f64(host(xt), gamma)
    full = xn @ oracle.round_bf16(W).astype(np.float64).T
    q_ref, g_ref = oracle.split_q_gate(full.astype(np.float32), heads, D)
    bar = 1e-2
    assert relerr(host(q), q_ref) <= bar and relerr(host(g), g_ref) <= bar
    # residual
    N2 = 1024
    W2 = oracle.normal((N2, K), 733, 0.0, 0.02)
    r = oracle.normal((M, N2), 734)
    w2 = qw.Weight.pack(ctx, W2, qw.WFMT_BF16)
    y = dev(r)
    qw.linear(ctx, w2, xt, y, residual=y)
    torch.cuda.synchronize()
    ref = oracle.linear_f64(oracle.round_bf16(W2), host(xt)) + r
    assert relerr(host(y), ref) <= 2e-5


@pytest.mark.parametrize("M", [33, 128, 300])
def test_gemm_lmhead_argmax(qw, ctx, oracle, M):
    V, K = 20000, 1024
    E = oracle.normal((V, K), 740, 0.0, 0.02)
    h = oracle.normal((M, K), 741 + M)
    Eb, hb = oracle.to_bf16(E), oracle.to_bf16(h)
    w = qw.Weight.pack(ctx, Eb, qw.WFMT_BF16, src_code=qw.BF16)
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    mx = torch.empty(M, device="cuda")
    qw.lmhead_argmax(ctx, w, dev(oracle.from_bf16(hb), torch.bfloat16), ids, mx)
    torch.cuda.synchronize()
    ref_ids, ref_max = oracle.lmhead_argmax_bf16(Eb, hb)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    np.testing.assert_allclose(mx.cpu().numpy(), ref_max, rtol=1e-4, atol=1e-5)


def test_gemm_repeatable(qw, ctx, oracle):
    M, N, K = 512, 1024, 1024
    w = qw.Weight.pack(ctx, oracle.normal((N, K), 750, 0.0, 0.02), qw.WFMT_BF16)
    xt = dev(oracle.normal((M, K), 751), torch.bfloat16)
    ys = torch.empty(5, M, N, device="cuda")
    for i in range(5):
        qw.linear(ctx, w, xt, ys[i])
    torch.cuda.synchronize()
    got = ys.cpu().numpy()
    assert (got == got[0][None]).all()


# ---------------------------------------------------------------------------
# INT8 weights (per-row scales): INT8 units in LDS, exact f16 conversion in
# registers, f16 MFMA, scale in the epilogue.  Bar: <= 1e-3 normwise against
# dequantize-then-multiply of the same q, s and activations (FP64 here, so
# only FP32 accumulation error remains: <= 2e-5 in practice).
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("xname", ["f16", "bf16"])
@pytest.mark.parametrize("M,N,K", [(33, 40, 64), (130, 1024, 1024), (300, 1032, 2048), (517, 4096, 1024)])
def test_gemm_int8_parity(qw, ctx, oracle, relerr, xname, M, N, K):
    W = oracle.normal((N, K), 800 + N, 0.0, 0.02)
    x = oracle.normal((M, K), 801 + M)
    w = qw.Weight.pack(ctx, W, qw.WFMT_INT8)
    q, sc = w.unpack()
    xt = dev(x, torch.float16 if xname == "f16" else torch.bfloat16)
    y = torch.empty(M, N, device="cuda")
    qw.linear(ctx, w, xt, y)
    torch.cuda.synchronize()
    xs = host(xt)
    assert relerr(host(y), oracle.linear_int8_f64(q, sc, xs)) <= 2e-5
    assert relerr(host(y), oracle.linear_int8(q, sc, xs)) <= 1e-3


def test_gemm_int8_exact(qw, ctx, oracle):
    """Integer activations and power-of-two scales: every product and partial
    sum is an exactly representable FP32 integer, so the GEMM must equal the
    FP64 result bit for bit (a dropped k, a wrong row or a mis-converted byte
    shows up as an integer error)."""
    M, N, K = 200, 512, 1024
    q = oracle.int8_uniform((N, K), 810)
    sc = np.float32(2.0) ** (-(np.arange(N) % 7)).astype(np.float32)
    x = np.round(oracle.normal((M, K), 811) * 2.0).clip(-4, 4).astype(np.float32)
    w = qw.Weight.pack(ctx, q, qw.WFMT_INT8, scales=sc)
    y = torch.empty(M, N, device="cuda")
    qw.linear(ctx, w, dev(x, torch.float16), y)
    torch.cuda.synchronize()
    ref = (x.astype(np.float64) @ q.astype(np.float64).T) * sc.astype(np.float64)[None, :]
    assert np.array_equal(host(y), ref.astype(np.float32))


@pytest.mark.parametrize("ydt", ["bf16", "f32"])
def test_gemm_int8_epilogues(qw, ctx, oracle, relerr, ydt):
    """GLU (gate/up pairs with their own scales), RMSNorm prologue (F16 copy
    in the workspace), residual add and the Q/gate split on INT8 weights."""
    ydtype = torch.bfloat16 if ydt == "bf16" else torch.float32
    # FP32 outputs: the north-star INT8 bar (the RMSNorm prologue feeds the
    # GEMM an F16 copy of the normalized activations, ~2.5e-4 normwise);
    # BF16 outputs add one output rounding
    bar_y = 4e-3 if ydt == "bf16" else 1e-3
    M, H, I = 150, 1024, 1024
    G = oracle.normal((I, H), 820, 0.0, 0.02)
    U = oracle.normal((I, H), 821, 0.0, 0.02)
    gamma = oracle.normal((H,), 822, 0.0, 0.02)
    x = oracle.normal((M, H), 823)
    gu = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_INT8)
    qgu, sgu = gu.unpack()
    xt = dev(x, torch.float16)
    h = torch.empty(M, I, device="cuda", dtype=ydtype)
    qw.linear(ctx, gu, xt, h, gamma=dev(gamma))
    torch.cuda.synchronize()
    xn = oracle.rmsnorm_f64(host(xt), gamma)
    g = oracle.linear_int8_f64(qgu[:I], sgu[:I], xn)
    u = oracle.linear_int8_f64(qgu[I:], sgu[I:], xn)
    assert relerr(host(h), g / (1.0 + np.exp(-g)) * u) <= bar_y
    # residual
    W2 = oracle.normal((H, I), 824, 0.0, 0.02)
    r = oracle.normal((M, H), 825)
    w2 = qw.Weight.pack(ctx, W2, qw.WFMT_INT8)
    q2, s2 = w2.unpack()
    hin = dev(oracle.normal((M, I), 826), torch.float16)
    y = dev(r, ydtype)
    ref = oracle.linear_int8_f64(q2, s2, host(hin)) + host(y)
    qw.linear(ctx, w2, hin, y, residual=y)
    torch.cuda.synchronize()
    assert relerr(host(y), ref) <= bar_y
    # Q/gate split
    heads, D = 4, 256
    W3 = oracle.normal((2 * heads * D, H), 827, 0.0, 0.02)
    w3 = qw.Weight.pack(ctx, W3, qw.WFMT_INT8)
    q3, s3 = w3.unpack()
    qo = torch.empty(M, heads * D, device="cuda", dtype=ydtype)
    go = torch.empty(M, heads * D, device="cuda", dtype=ydtype)
    qw.linear(ctx, w3, xt, qo, y2=go, split_period=D)
    torch.cuda.synchronize()
    full = oracle.linear_int8_f64(q3, s3, host(xt))
    q_ref, g_ref = oracle.split_q_gate(full.astype(np.float32), heads, D)
    assert relerr(host(qo), q_ref) <= bar_y and relerr(host(go), g_ref) <= bar_y


@pytest.mark.parametrize("M", [33, 128, 300])
def test_gemm_int8_lmhead_argmax(qw, ctx, oracle, M):
    V, K = 20000, 1024
    E = oracle.normal((V, K), 830, 0.0, 0.02)
    h = oracle.normal((M, K), 831 + M)
    w = qw.Weight.pack(ctx, E, qw.WFMT_INT8)
    q, sc = w.unpack()
    ht = dev(h, torch.float16)
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    qw.lmhead_argmax(ctx, w, ht, ids)
    torch.cuda.synchronize()
    ref_ids, _ = oracle.lmhead_argmax_int8(q, sc, host(ht))
    assert np.array_equal(ids.cpu().numpy(), ref_ids)


@pytest.mark.parametrize("K,M", [(2048, 1024), (3584, 1024), (3584, 384), (2048, 700), (3584, 700)])
def test_gemm_splitk_default_route(qw, oracle, relerr, K, M):
    """The default routing of a 1024-row projection at a few hundred to 1024
    tokens (the prefill out / down projections): 64-row blocks with the K
    range split over 2-4 workgroups per tile (M=700: a ragged last block), partial tiles handed to the last split, which
    adds them in split order and runs the residual epilogue.  Same FP32 bar
    as the unsplit GEMM (2e-5 vs FP64 on the stored operands); two calls in a
    row give identical results (the arrival counters return to zero)."""
    N = 1024
    c = qw.Context(0)
    W = oracle.normal((N, K), 760 + K, 0.0, 0.02)
    x = oracle.normal((M, K), 761)
    r = oracle.normal((M, N), 762)
    w = qw.Weight.pack(c, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    ys = []
    for _ in range(2):
        y = dev(r)
        qw.linear(c, w, xt, y, residual=y)
        ys.append(y)
    torch.cuda.synchronize()
    ref = oracle.linear_f64(oracle.round_bf16(W), host(xt)) + r
    assert relerr(host(ys[0]), ref) <= 2e-5
    assert torch.equal(ys[0], ys[1])
    del w
    c.close()
