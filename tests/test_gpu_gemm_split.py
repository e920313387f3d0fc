"""GPU parity of the split-K direct-A GEMM (qw_gemm_da.hip: S workgroups per
256 x 128 block store FP32 partial tiles, gemm_da_reduce sums them in split
order and runs the epilogue), forced to each K split count the shapes allow
(QW_GEMM_DA_SPLIT), against FP64 on the stored BF16 operands and against the
route without it (QW_GEMM_DA_SPLIT=0), plus bit-identical repeats.

Shapes: the 1024-row down projection (K = 3584) and out projection (K = 2048)
with the residual epilogue at 520..2048 tokens, the 7168-row gate/up GLU
(K = 1024), and the 4096-row Q+gate with the split epilogue.  Bars: <= 2e-5
normwise vs FP64 on the stored operands (FP32 output; the split regroups FP32
sums only), <= 1e-5 vs the other route; 1e-4 for the GLU (SiLU of sums).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


@pytest.fixture(scope="module")
def ctx_s(qw):
    """Contexts by forced split count, created on demand (0: the split route off)."""
    import os
    made = {}

    def get(S):
        if S not in made:
            old = os.environ.get("QW_GEMM_DA_SPLIT")
            os.environ["QW_GEMM_DA_SPLIT"] = str(S)
            try:
                made[S] = qw.Context(0)
            finally:
                if old is None:
                    os.environ.pop("QW_GEMM_DA_SPLIT", None)
                else:
                    os.environ["QW_GEMM_DA_SPLIT"] = old
        return made[S]
    yield get
    for c in made.values():
        c.close()


@pytest.mark.parametrize("K,M,S", [(3584, 1024, 2), (3584, 1024, 7), (3584, 1024, 14), (3584, 520, 4),
                                   (3584, 2048, 4), (2048, 1024, 8), (2048, 600, 4), (2048, 1536, 2)])
def test_split_residual_1024_rows(qw, ctx_s, oracle, relerr, K, M, S):
    ctx = ctx_s(S)
    W = oracle.normal((1024, K), 7100 + K, 0.0, 0.02)
    x = oracle.normal((M, K), 7101 + M)
    r = oracle.normal((M, 1024), 7102)
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    y = dev(r)
    qw.linear(ctx, w, xt, y, residual=y)
    y2 = dev(r)
    qw.linear(ctx, w, xt, y2, residual=y2)
    c0 = ctx_s(0)
    w0 = qw.Weight.pack(c0, W, qw.WFMT_BF16)
    y0 = dev(r)
    qw.linear(c0, w0, xt, y0, residual=y0)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    assert torch.equal(y, y2), "repeat differs"
    ref = oracle.linear_f64(oracle.round_bf16(W), host(xt)) + r
    assert relerr(host(y), ref) <= 2e-5
    assert relerr(host(y), host(y0).astype(np.float64)) <= 1e-5


@pytest.mark.parametrize("M,S", [(600, 2), (520, 4)])
def test_split_glu(qw, ctx_s, oracle, relerr, M, S):
    ctx = ctx_s(S)
    I, H = 3584, 1024
    G = oracle.normal((I, H), 7130, 0.0, 0.02)
    U = oracle.normal((I, H), 7131, 0.0, 0.02)
    x = oracle.normal((M, H), 7133 + M)
    w = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    h = torch.empty(M, I, device="cuda")
    qw.linear(ctx, w, xt, h)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    xs = host(xt).astype(np.float64)
    g = xs @ oracle.round_bf16(G).astype(np.float64).T
    u = xs @ oracle.round_bf16(U).astype(np.float64).T
    assert relerr(host(h), g / (1.0 + np.exp(-g)) * u) <= 1e-4


def test_split_q_gate(qw, ctx_s, oracle, relerr):
    """Q+gate (4096 rows interleaved per 256-dim head) with the split epilogue, S = 4."""
    ctx = ctx_s(4)
    heads, D, K, M = 8, 256, 1024, 640
    W = oracle.normal((2 * heads * D, K), 7140, 0.0, 0.02)
    x = oracle.normal((M, K), 7141)
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    q = torch.empty(M, heads * D, device="cuda")
    g = torch.empty(M, heads * D, device="cuda")
    qw.linear(ctx, w, xt, q, y2=g, split_period=D)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    full = oracle.linear_f64(oracle.round_bf16(W), host(xt))
    q_ref, g_ref = oracle.split_q_gate(full.astype(np.float32), heads, D)
    assert relerr(host(q), q_ref) <= 1e-5 and relerr(host(g), g_ref) <= 1e-5
