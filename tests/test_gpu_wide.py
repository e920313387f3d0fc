"""GPU parity of the weight-stationary projection kernel (qw_wide.hip), which
takes 17..512 tokens on BF16 weights (BF16 activations) and INT8 weights (F16
activations).

The contexts here switch the MFMA GEMM off (QW_GEMM_MIN_M) so every call runs
the weight-stationary kernel, at token counts that exercise each token-tile
count (2, 4, 8 tiles of 16) and token-group split (up to 8 groups of at
most 128 tokens), ragged last tiles, odd tile counts (the last
block of two tiles half empty), a partial last tile (N = 24), every K-split
/ workgroup shape the planner can pick (forced through QW_WIDE_S and
QW_WIDE_CFG), and every epilogue: residual (FP32 and BF16, in place), GLU
with and without the RMSNorm prologue (per-call gamma and a folded norm
weight), the Q/gate split, and the element-wise store path of unaligned
outputs.

Bars as for the other projection kernels: BF16 weights <= 2e-5 normwise vs
FP64 on the stored operands (FP32 output), and <= 1e-2 with the RMSNorm
prologue (the normalized activations are rounded to BF16 for the MFMA);
INT8 weights <= 1e-3 normwise vs the reference's dequant-then-matmul
(mlp_cuda.cu:158-180) and per element on outputs above a tenth of the RMS.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def _elementwise(got, ref, bar):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    floor = np.sqrt(np.mean(ref ** 2)) / 10
    assert np.all(np.abs(got - ref) <= bar * np.maximum(np.abs(ref), floor))


def _ctx(qw, **env):
    """A context created with the given QW_* settings (read at qw_init)."""
    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return qw.Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.fixture(scope="module")
def wctx(qw):
    c = _ctx(qw, QW_GEMM_MIN_M=1 << 30)
    yield c
    torch.cuda.synchronize()
    c.close()


MS = [17, 32, 33, 64, 100, 128, 129, 200, 256, 300, 384, 512]


@pytest.mark.parametrize("M", MS)
@pytest.mark.parametrize("N,K", [(1024, 2048), (8192, 1024), (1040, 1024), (24, 1024)])
def test_bf16_plain(qw, wctx, oracle, relerr, N, K, M):
    W = oracle.normal((N, K), 3000 + N + K, 0.0, 0.02)
    x = oracle.normal((M, K), 3001 + M)
    w = qw.Weight.pack(wctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    y = torch.full((M, N), 7.0, device="cuda")
    qw.linear(wctx, w, xt, y)
    torch.cuda.synchronize()
    assert wctx.device_error() == 0
    assert relerr(host(y), oracle.linear_f64(oracle.round_bf16(W), host(xt))) <= 2e-5


@pytest.mark.parametrize("M", [17, 64, 128, 256, 512])
@pytest.mark.parametrize("rdt", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_bf16_residual_down(qw, wctx, oracle, relerr, M, rdt):
    """down (1024 x 3584, many K splits) with the residual added in place."""
    W = oracle.normal((1024, 3584), 3010, 0.0, 0.02)
    x = oracle.normal((M, 3584), 3011 + M)
    r = oracle.normal((M, 1024), 3012)
    w = qw.Weight.pack(wctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    y = dev(r, rdt)
    r_used = host(y)
    qw.linear(wctx, w, xt, y, residual=y)
    torch.cuda.synchronize()
    ref = oracle.linear_f64(oracle.round_bf16(W), host(xt)) + r_used
    assert relerr(host(y), ref) <= (2e-5 if rdt == torch.float32 else 8e-3)


@pytest.fixture(scope="module")
def wctx_sep_norm(qw):
    """The RMSNorm prologue as a separate normalization launch instead of
    inside the weight-stationary kernel."""
    c = _ctx(qw, QW_GEMM_MIN_M=1 << 30, QW_WIDE_NORM_SEP=1)
    yield c
    torch.cuda.synchronize()
    c.close()


@pytest.mark.parametrize("M", [20, 48, 128, 256, 384, 512])
@pytest.mark.parametrize("norm", ["none", "gamma", "folded", "gamma_sep", "folded_sep"])
def test_bf16_glu(qw, wctx, wctx_sep_norm, oracle, relerr, M, norm):
    if norm.endswith("_sep"):
        wctx, norm = wctx_sep_norm, norm[: -len("_sep")]
    I, H = 3584, 1024
    G = oracle.normal((I, H), 3020, 0.0, 0.02)
    U = oracle.normal((I, H), 3021, 0.0, 0.02)
    gamma = oracle.normal((H,), 3022, 0.0, 0.02)
    x = oracle.normal((M, H), 3023 + M)
    w = qw.Weight.pack_glu(wctx, G, U, qw.WFMT_BF16)
    if norm == "folded":
        w.fold_norm(dev(gamma))
    xt = dev(x, torch.bfloat16)
    h = torch.empty(M, I, device="cuda")
    qw.linear(wctx, w, xt, h, gamma=dev(gamma) if norm == "gamma" else None, norm=norm == "folded")
    torch.cuda.synchronize()
    xs = oracle.rmsnorm_f64(host(xt), gamma) if norm != "none" else host(xt).astype(np.float64)
    g = xs @ oracle.round_bf16(G).astype(np.float64).T
    u = xs @ oracle.round_bf16(U).astype(np.float64).T
    ref = g / (1.0 + np.exp(-g)) * u
    assert relerr(host(h), ref) <= (1e-2 if norm != "none" else 1e-4)


@pytest.mark.parametrize("M", [40, 128])
def test_bf16_split_q_gate(qw, wctx, oracle, relerr, M):
    heads, D, K = 8, 256, 1024
    W = oracle.normal((2 * heads * D, K), 3030, 0.0, 0.02)
    x = oracle.normal((M, K), 3031)
    w = qw.Weight.pack(wctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    q = torch.empty(M, heads * D, device="cuda")
    g = torch.empty(M, heads * D, device="cuda")
    qw.linear(wctx, w, xt, q, y2=g, split_period=D)
    torch.cuda.synchronize()
    full = oracle.linear_f64(oracle.round_bf16(W), host(xt))
    q_ref, g_ref = oracle.split_q_gate(full.astype(np.float32), heads, D)
    assert relerr(host(q), q_ref) <= 1e-5 and relerr(host(g), g_ref) <= 1e-5


def test_bf16_unaligned_output(qw, wctx, oracle, relerr):
    """A row pitch that is not a multiple of 4 takes the element-wise stores
    (residual read from global memory)."""
    M, N, K = 50, 1024, 2048
    W = oracle.normal((N, K), 3040, 0.0, 0.02)
    x = oracle.normal((M, K), 3041)
    r = oracle.normal((M, N), 3042)
    w = qw.Weight.pack(wctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    ybuf = torch.zeros(M, N + 3, device="cuda")
    y = ybuf[:, :N]
    y.copy_(dev(r))
    qw.linear(wctx, w, xt, y, residual=y)
    torch.cuda.synchronize()
    ref = oracle.linear_f64(oracle.round_bf16(W), host(xt)) + r
    assert relerr(host(y), ref) <= 2e-5
    assert torch.all(ybuf[:, N:] == 0)


@pytest.mark.parametrize("M", [17, 32, 64, 128, 256, 384, 512])
@pytest.mark.parametrize("N,K", [(1024, 3584), (6144, 1024), (512, 1024), (1024, 2048)])
def test_int8_plain(qw, wctx, oracle, relerr, N, K, M):
    q = oracle.int8_uniform((N, K), 3100 + N + K)
    s = oracle.uniform((N,), 3101 + N, 1e-3, 2e-2)
    x = oracle.normal((M, K), 3102 + M)
    w = qw.Weight.pack(wctx, q, qw.WFMT_INT8, scales=s)
    xt = dev(x, torch.float16)
    y = torch.empty(M, N, device="cuda")
    qw.linear(wctx, w, xt, y)
    torch.cuda.synchronize()
    ref = oracle.linear_int8(q, s, host(xt))
    assert relerr(host(y), ref) <= 1e-3
    _elementwise(host(y), ref, 1e-3)


@pytest.mark.parametrize("M", [24, 128, 256, 512])
def test_int8_glu_and_residual(qw, wctx, oracle, relerr, M):
    I, H = 3584, 1024
    qg = oracle.int8_uniform((I, H), 3110)
    qu = oracle.int8_uniform((I, H), 3111)
    sg = oracle.uniform((I,), 3112, 1e-3, 2e-2)
    su = oracle.uniform((I,), 3113, 1e-3, 2e-2)
    qd = oracle.int8_uniform((H, I), 3114)
    sd = oracle.uniform((H,), 3115, 1e-3, 2e-2)
    x = oracle.normal((M, H), 3116)
    r = oracle.normal((M, H), 3117)
    gu = qw.Weight.pack_glu(wctx, qg, qu, qw.WFMT_INT8, gate_scales=sg, up_scales=su)
    dn = qw.Weight.pack(wctx, qd, qw.WFMT_INT8, scales=sd)
    xt = dev(x, torch.float16)
    h = torch.empty(M, I, device="cuda", dtype=torch.float16)
    qw.linear(wctx, gu, xt, h)
    y = dev(r)   # FP32: the INT8 down outputs reach ~6e4
    r_used = host(y)
    qw.linear(wctx, dn, h, y, residual=y)
    torch.cuda.synchronize()
    xs = host(xt)
    g = oracle.linear_int8(qg, sg, xs).astype(np.float64)
    u = oracle.linear_int8(qu, su, xs).astype(np.float64)
    h_ref = g / (1.0 + np.exp(-g)) * u
    assert relerr(host(h), h_ref) <= 1e-3
    y_ref = oracle.linear_int8(qd, sd, host(h)).astype(np.float64) + r_used
    assert relerr(host(y), y_ref) <= 1e-3


@pytest.mark.parametrize("cfg", [1, 2, 3])
@pytest.mark.parametrize("S", [1, 2, 3, 7])
def test_forced_shapes(qw, oracle, relerr, cfg, S):
    """Every workgroup shape (4x1, 2x2, 1x4 blocks x waves) at several K
    splits, including uneven ones, on BF16 and INT8 weights."""
    c = _ctx(qw, QW_GEMM_MIN_M=1 << 30, QW_WIDE_CFG=cfg, QW_WIDE_S=S)
    try:
        M, N, K = 40, 2080, 2048
        W = oracle.normal((N, K), 3200, 0.0, 0.02)
        x = oracle.normal((M, K), 3201)
        w = qw.Weight.pack(c, W, qw.WFMT_BF16)
        xt = dev(x, torch.bfloat16)
        y = torch.empty(M, N, device="cuda")
        qw.linear(c, w, xt, y)
        q = oracle.int8_uniform((N, K), 3202)
        s = oracle.uniform((N,), 3203, 1e-3, 2e-2)
        w8 = qw.Weight.pack(c, q, qw.WFMT_INT8, scales=s)
        x16 = dev(x, torch.float16)
        y8 = torch.empty(M, N, device="cuda")
        qw.linear(c, w8, x16, y8)
        torch.cuda.synchronize()
        assert relerr(host(y), oracle.linear_f64(oracle.round_bf16(W), host(xt))) <= 2e-5
        assert relerr(host(y8), oracle.linear_int8(q, s, host(x16))) <= 1e-3
        del w, w8
    finally:
        torch.cuda.synchronize()
        c.close()


def test_repeatable_and_graph_safe(qw, wctx, oracle):
    """Bit-identical results over repeated calls (fixed reduction orders, the
    split-K counters return to zero), eager and replayed from a graph."""
    M, N, K = 128, 1024, 3584
    W = oracle.normal((N, K), 3300, 0.0, 0.02)
    x = oracle.normal((M, K), 3301)
    w = qw.Weight.pack(wctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    y0 = torch.empty(M, N, device="cuda")
    qw.linear(wctx, w, xt, y0)
    torch.cuda.synchronize()
    y = torch.empty(M, N, device="cuda")
    for _ in range(20):
        y.zero_()
        qw.linear(wctx, w, xt, y)
        torch.cuda.synchronize()
        assert torch.equal(y, y0)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        g = qw.Graph(wctx, stream)
        with g:
            qw.linear(wctx, w, xt, y, stream=stream)
        for _ in range(5):
            y.zero_()
            g.launch(stream)
            stream.synchronize()
            assert torch.equal(y, y0)
    torch.cuda.synchronize()


@pytest.mark.parametrize("M", [24, 128, 300])
@pytest.mark.parametrize("sep", [False, True])
def test_int8_glu_norm(qw, wctx, wctx_sep_norm, oracle, relerr, M, sep):
    """INT8 gate/up with the RMSNorm prologue (F16 activations): against the
    dequant-then-matmul of the FP64-normalized activations."""
    c = wctx_sep_norm if sep else wctx
    I, H = 3584, 1024
    qg = oracle.int8_uniform((I, H), 3400)
    qu = oracle.int8_uniform((I, H), 3401)
    sg = oracle.uniform((I,), 3402, 1e-3, 2e-2)
    su = oracle.uniform((I,), 3403, 1e-3, 2e-2)
    gamma = oracle.normal((H,), 3404, 0.0, 0.02)
    x = oracle.normal((M, H), 3405)
    gu = qw.Weight.pack_glu(c, qg, qu, qw.WFMT_INT8, gate_scales=sg, up_scales=su)
    xt = dev(x, torch.float16)
    h = torch.empty(M, I, device="cuda")
    qw.linear(c, gu, xt, h, gamma=dev(gamma))
    torch.cuda.synchronize()
    xs = oracle.rmsnorm_f64(host(xt), gamma)
    g = oracle.linear_int8_f64(qg, sg, xs)
    u = oracle.linear_int8_f64(qu, su, xs)
    ref = g / (1.0 + np.exp(-g)) * u
    # the weights times (1 + gamma), or the normalized activations, are
    # rounded to F16 for the MFMA (2^-11 per term)
    assert relerr(host(h), ref) <= 2e-3


@pytest.mark.parametrize("M", [17, 40, 65, 100, 128, 256])
@pytest.mark.parametrize("fmt", ["bf16", "int8", "int8_bf16x"])
def test_lmhead_argmax_odd_vocab(qw, ctx, oracle, fmt, M):
    """The weight-stationary lm_head argmax on a vocabulary of 627 tiles (the
    last block holds one tile, its last 8 rows past the end): ids equal the
    oracle's (LMHead::forward + Sampler::sample_greedy, lm_head.cpp:24-39,
    sampler.cpp:41-43) where its top-2 gap is clear, the maximum planted in
    the last row is found, and exact ties resolve to the lowest row.
    "int8_bf16x": INT8 weights with BF16 activations (converted to f16 in
    LDS, exact for these magnitudes)."""
    V, K = 10024, 1024
    E = oracle.normal((V, K), 3500, 0.0, 0.02)
    h = oracle.normal((M, K), 3501)
    hb = oracle.round_f16(h) if fmt == "int8" else oracle.round_bf16(h)
    c = 0.0625
    E[V - 1] = c * np.sign(hb[0])        # token 0: unique maximum in the last row
    E[[4100, 4101, 9999]] = c * np.sign(hb[1])  # token 1: exact tie -> 4100
    Eb = oracle.round_bf16(E)
    if fmt == "bf16":
        w = qw.Weight.pack(ctx, Eb, qw.WFMT_BF16)
        x = dev(hb, torch.bfloat16)
        logits = hb.astype(np.float64) @ Eb.astype(np.float64).T
    else:
        w = qw.Weight.pack(ctx, Eb, qw.WFMT_INT8)
        q, s = w.unpack()
        x = dev(hb, torch.float16 if fmt == "int8" else torch.bfloat16)
        logits = (hb.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)[None, :]
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    qw.lmhead_argmax(ctx, w, x, ids)
    torch.cuda.synchronize()
    got = ids.cpu().numpy()
    assert int(got[0]) == V - 1
    assert int(got[1]) == 4100
    for t in range(2, M):
        srt = np.sort(logits[t])
        if srt[-1] - srt[-2] > 1e-3:
            assert int(got[t]) == int(np.argmax(logits[t])), t


@pytest.mark.parametrize("M", [65, 100, 128])
def test_lmhead_argmax_activation_stationary_matches(qw, ctx, oracle, M):
    """BF16 E at 65..128 tokens takes the activation-stationary lm_head argmax
    (E through an LDS ring once, each wave holding a token tile): its ids and
    winning logits equal the weight-stationary kernel's (a context made with
    QW_ARGMAX_AS=0) bit for bit, on a vocabulary with an odd tile count, twice
    in a row (keys and the completion count return to zero)."""
    import os
    V, K = 10024, 1024
    E = oracle.round_bf16(oracle.normal((V, K), 3600, 0.0, 0.02))
    h = oracle.normal((M, K), 3601 + M)
    os.environ["QW_ARGMAX_AS"] = "0"
    try:
        c2 = qw.Context(0)
    finally:
        del os.environ["QW_ARGMAX_AS"]
    try:
        w1 = qw.Weight.pack(ctx, E, qw.WFMT_BF16)
        w2 = qw.Weight.pack(c2, E, qw.WFMT_BF16)
        x = dev(h, torch.bfloat16)
        for rep in range(2):
            ids1 = torch.full((M,), -1, dtype=torch.int32, device="cuda")
            mx1 = torch.empty(M, device="cuda")
            qw.lmhead_argmax(ctx, w1, x, ids1, mx1)
            ids2 = torch.full((M,), -1, dtype=torch.int32, device="cuda")
            mx2 = torch.empty(M, device="cuda")
            qw.lmhead_argmax(c2, w2, x, ids2, mx2)
            torch.cuda.synchronize()
            assert torch.equal(ids1, ids2), rep
            assert torch.equal(mx1, mx2), rep
            assert int(ids1.min()) >= 0
        assert ctx.device_error() == 0 and c2.device_error() == 0
    finally:
        c2.close()


def test_splitk_partials_return_to_sentinel(qw, wctx, oracle):
    """The split-K partials region holds a sentinel between launches; every
    finishing workgroup writes it back over the words it consumed.  Launches
    with different plans (split counts, token groups, units per workgroup,
    with and without the norm prologue) reuse the same words in different
    layouts, so a word left holding a partial would be taken for a partner's
    fresh one by a later launch.  The same calls in two different orders, on
    one context, must give the same outputs bit for bit."""
    rng = np.random.default_rng(4200)
    cases = []
    for N, K, glu in ((1024, 3584, False), (1024, 2048, False), (3584, 1024, True)):
        if glu:
            w = qw.Weight.pack_glu(wctx, oracle.normal((N, K), 4201, 0.0, 0.02), oracle.normal((N, K), 4202, 0.0, 0.02),
                                   qw.WFMT_BF16)
        else:
            w = qw.Weight.pack(wctx, oracle.normal((N, K), 4203 + N + K, 0.0, 0.02), qw.WFMT_BF16)
        for M in (17, 32, 64, 100, 128, 256):
            x = dev(rng.standard_normal((M, K)).astype(np.float32), torch.bfloat16)
            gam = dev(rng.standard_normal(K).astype(np.float32) * 0.05) if glu else None
            cases.append((w, x, gam, N, M))

    def run(order):
        outs = {}
        for i in order:
            w, x, gam, N, M = cases[i]
            y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
            qw.linear(wctx, w, x, y, gamma=gam)
            outs[i] = y
        torch.cuda.synchronize()
        return outs

    a = run(range(len(cases)))
    b = run(reversed(range(len(cases))))
    c = run(rng.permutation(len(cases)))
    assert wctx.device_error() == 0
    for i in range(len(cases)):
        assert torch.equal(a[i], b[i]), i
        assert torch.equal(a[i], c[i]), i
