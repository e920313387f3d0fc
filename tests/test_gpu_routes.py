"""GPU parity of the projections on the DEFAULT routes (no forced kernel) at
the token counts where the route changes, and of the token-embedding gather.

Route cases (qw_linear's routing by weight rows and tokens):
  * 8224-row stacked QKV+Z+a+b at 512 tokens (256-row GEMM blocks), 4096 rows
    at 1024 tokens with the Q/gate split (64-row blocks), 5120 rows at 768
    tokens (64-row blocks), the 1024-row out projection at 768 tokens with the
    residual (64-row blocks with split-K), the 7168-row gate/up GLU at 512 and
    1024 tokens with and without the RMSNorm prologue;
  * config 3 (INT8 weight-only, F16 activations) at 32 and 128 tokens on every
    layer shape, including K = 2048 (out / O) and the 512-row K / V, which run
    the small-M kernels.
Bars: BF16 <= 1e-2 normwise vs FP64 on the unrounded weights and <= 2e-5 vs
FP64 on the stored operands (FP32 output); INT8 <= 1e-3 normwise vs the
reference's dequant-then-matmul (mlp_cuda.cu:158-180 with the scale applied
to the dot product), plus a per-element bar of 1e-3 on every output whose
magnitude is at least a tenth of the output's RMS.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def _elementwise(got, ref, bar):
    """|got - ref| <= bar * |ref| on outputs with |ref| >= rms(ref) / 10, and
    <= bar * rms(ref) / 10 below that floor."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    floor = np.sqrt(np.mean(ref ** 2)) / 10
    assert np.all(np.abs(got - ref) <= bar * np.maximum(np.abs(ref), floor))


@pytest.mark.parametrize("N,M", [(8224, 512), (5120, 768), (4096, 1024), (8224, 256), (5120, 320)])
def test_default_route_stacked(qw, ctx, oracle, relerr, N, M):
    W = oracle.normal((N, 1024), 1100 + N, 0.0, 0.02)
    x = oracle.normal((M, 1024), 1101 + M)
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    y = torch.empty(M, N, device="cuda")
    qw.linear(ctx, w, xt, y)
    torch.cuda.synchronize()
    xs = host(xt)
    assert relerr(host(y), oracle.linear_f64(oracle.round_bf16(W), xs)) <= 2e-5
    assert relerr(host(y), oracle.linear_f64(W, xs)) <= 1e-2


@pytest.mark.parametrize("M", [1024, 256])
def test_default_route_split_q_gate(qw, ctx, oracle, relerr, M):
    """Q+gate (4096 rows, interleaved per 256-dim head) with the split epilogue."""
    heads, D, K = 8, 256, 1024
    W = oracle.normal((2 * heads * D, K), 1110, 0.0, 0.02)
    x = oracle.normal((M, K), 1111)
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    q = torch.empty(M, heads * D, device="cuda")
    g = torch.empty(M, heads * D, device="cuda")
    qw.linear(ctx, w, xt, q, y2=g, split_period=D)
    torch.cuda.synchronize()
    full = oracle.linear_f64(oracle.round_bf16(W), host(xt))
    q_ref, g_ref = oracle.split_q_gate(full.astype(np.float32), heads, D)
    assert relerr(host(q), q_ref) <= 1e-5 and relerr(host(g), g_ref) <= 1e-5


@pytest.mark.parametrize("M,K", [(768, 2048), (1024, 3584), (384, 3584), (512, 2048)])
def test_default_route_residual_1024_rows(qw, ctx, oracle, relerr, M, K):
    """out / O (K = 2048) and down (K = 3584): 1024 rows, residual in place."""
    W = oracle.normal((1024, K), 1120 + K, 0.0, 0.02)
    x = oracle.normal((M, K), 1121 + M)
    r = oracle.normal((M, 1024), 1122)
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    y = dev(r)
    qw.linear(ctx, w, xt, y, residual=y)
    torch.cuda.synchronize()
    ref = oracle.linear_f64(oracle.round_bf16(W), host(xt)) + r
    assert relerr(host(y), ref) <= 2e-5


@pytest.mark.parametrize("M", [512, 1024, 200])
@pytest.mark.parametrize("norm", [False, True])
def test_default_route_glu(qw, ctx, oracle, relerr, M, norm):
    I, H = 3584, 1024
    G = oracle.normal((I, H), 1130, 0.0, 0.02)
    U = oracle.normal((I, H), 1131, 0.0, 0.02)
    gamma = oracle.normal((H,), 1132, 0.0, 0.02)
    x = oracle.normal((M, H), 1133)
    w = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    h = torch.empty(M, I, device="cuda")
    qw.linear(ctx, w, xt, h, gamma=dev(gamma) if norm else None)
    torch.cuda.synchronize()
    xs = oracle.rmsnorm_f64(host(xt), gamma) if norm else host(xt).astype(np.float64)
    g = xs @ oracle.round_bf16(G).astype(np.float64).T
    u = xs @ oracle.round_bf16(U).astype(np.float64).T
    ref = g / (1.0 + np.exp(-g)) * u
    # with the prologue the normalized activations are rounded to BF16
    assert relerr(host(h), ref) <= (1e-2 if norm else 1e-4)


# ----------------------------------------------------------------------------
# config 3: INT8 weight-only projections of one layer, default route
# ----------------------------------------------------------------------------

CFG3 = [("q_gate", 4096, 1024), ("k", 512, 1024), ("v", 512, 1024), ("o", 1024, 2048),
        ("qkv", 6144, 1024), ("z", 2048, 1024), ("out", 1024, 2048), ("down", 1024, 3584)]


@pytest.mark.parametrize("M", [1, 32, 128])
@pytest.mark.parametrize("name,N,K", CFG3, ids=[c[0] for c in CFG3])
def test_cfg3_int8_default_route(qw, ctx, oracle, relerr, name, N, K, M):
    q = oracle.int8_uniform((N, K), 1200 + N + K)
    s = oracle.uniform((N,), 1201 + N, 1e-3, 2e-2)
    x = oracle.normal((M, K), 1202 + M)
    w = qw.Weight.pack(ctx, q, qw.WFMT_INT8, scales=s)
    xt = dev(x, torch.float16)
    y = torch.empty(M, N, device="cuda")
    qw.linear(ctx, w, xt, y)
    torch.cuda.synchronize()
    xs = host(xt)
    ref = oracle.linear_int8(q, s, xs)        # FP32 dequant-then-matmul order
    assert relerr(host(y), ref) <= 1e-3
    _elementwise(host(y), ref, 1e-3)
    ref64 = oracle.linear_int8_f64(q, s, xs)
    assert relerr(host(y), ref64) <= 2e-5


@pytest.mark.parametrize("M", [32, 128])
def test_cfg3_int8_glu_default_route(qw, ctx, oracle, relerr, M):
    I, H = 3584, 1024
    qg = oracle.int8_uniform((I, H), 1210)
    qu = oracle.int8_uniform((I, H), 1211)
    sg = oracle.uniform((I,), 1212, 1e-3, 2e-2)
    su = oracle.uniform((I,), 1213, 1e-3, 2e-2)
    x = oracle.normal((M, H), 1214)
    w = qw.Weight.pack_glu(ctx, qg, qu, qw.WFMT_INT8, gate_scales=sg, up_scales=su)
    xt = dev(x, torch.float16)
    h = torch.empty(M, I, device="cuda")
    qw.linear(ctx, w, xt, h)
    torch.cuda.synchronize()
    xs = host(xt)
    g = oracle.linear_int8(qg, sg, xs).astype(np.float64)
    u = oracle.linear_int8(qu, su, xs).astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    assert relerr(host(h), ref) <= 1e-3
    _elementwise(host(h), ref, 1e-3)


# ----------------------------------------------------------------------------
# token-embedding gather (token_embedding_cuda.cu:28-58)
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("tdt", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_embedding_gather_full_vocab(qw, ctx, tdt):
    """Rows 0, V-1 and others of the 248320-row table are copied exactly; an
    out-of-range id (V, -1) gives a zero row and raises the device flag, which
    qw_device_error reads and clears."""
    V, H = 248320, 1024
    g = torch.Generator().manual_seed(77)
    table = torch.empty(V, H).normal_(0.0, 0.02, generator=g).to(tdt).cuda()
    good = [0, V - 1, 12345, 131072, 1]
    ids = torch.tensor(good, dtype=torch.int32, device="cuda")
    for odt in (torch.float32, torch.bfloat16):
        out = torch.full((len(good), H), 7.0, device="cuda", dtype=odt)
        qw.embedding_gather(ctx, table, ids, out)
        torch.cuda.synchronize()
        assert ctx.device_error() == 0
        assert torch.equal(out.float(), table[ids.long()].float().to(odt).float())
    bad = torch.tensor([V - 1, V, -1, 0], dtype=torch.int32, device="cuda")
    out = torch.full((4, H), 7.0, device="cuda")
    qw.embedding_gather(ctx, table, bad, out)
    torch.cuda.synchronize()
    assert ctx.device_error() == 1
    assert ctx.device_error() == 0          # read clears it
    assert torch.equal(out[0], table[V - 1].float())
    assert torch.equal(out[3], table[0].float())
    assert torch.count_nonzero(out[1:3]) == 0
    # a strided output (ld_out > hidden) leaves the gap untouched
    wide = torch.full((2, H + 64), 3.0, device="cuda")
    qw.embedding_gather(ctx, table, ids[:2], wide[:, :H], ld_out=H + 64)
    torch.cuda.synchronize()
    assert torch.equal(wide[:, :H], table[ids[:2].long()].float())
    assert torch.all(wide[:, H:] == 3.0)
