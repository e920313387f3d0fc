"""GPU parity of qw_layer_tail (out-projection + residual, then the post-norm
MLP + residual, on the FP32 residual stream; with QW_LAYER_TAIL=1 one launch
at decode sizes, by default the two calls) against the oracle's FP64
composition and against the two calls it replaces (qw_linear with the
residual epilogue, then qw_mlp_fused).

Bars: BF16 weights <= 1e-2 normwise vs FP64 on the BF16-rounded weights;
INT8 weights <= 1e-3 vs the dequant-then-matmul composition of the same q
and s with the kernel's F16 rounding of h; one launch vs the two calls
<= 1e-3 (the same math; the out-projection's K is summed in another grouping,
which can move a 16-bit rounding of h).  Every call must leave the device
error flag clear.  Reference: CudaLayer::forward (cuda_engine.cu:118-124).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

H, I, KO = 1024, 3584, 2048


@pytest.fixture(scope="module", params=["one", "two"])
def ctx(qw, request):
    """A context with the one-launch route on (QW_LAYER_TAIL=1: the first
    gate/up workgroups run the out-projection; opt-in, it measured slower
    than the two launches in the decode step), and the default context (the
    two calls)."""
    import os
    env = {"QW_LAYER_TAIL": "1" if request.param == "one" else "0"}
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        c = qw.Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    yield c
    c.close()


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def _bf16_case(qw, ctx, oracle, seed):
    Wo = oracle.normal((H, KO), seed, 0.0, 0.02)
    G = oracle.normal((I, H), seed + 1, 0.0, 0.02)
    U = oracle.normal((I, H), seed + 2, 0.0, 0.02)
    D = oracle.normal((H, I), seed + 3, 0.0, 0.02)
    gam = oracle.normal((H,), seed + 4, 0.0, 0.05)
    w = (qw.Weight.pack(ctx, Wo, qw.WFMT_BF16), qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16),
         qw.Weight.pack(ctx, D, qw.WFMT_BF16))
    return (Wo, G, U, D, gam), w


def _ref_bf16(oracle, mats, core, x):
    Wo, G, U, D, gam = mats
    xm = x.astype(np.float64) + oracle.linear_f64(oracle.round_bf16(Wo), core)
    return oracle.mlp_block_f64(oracle.round_bf16(G), oracle.round_bf16(U), oracle.round_bf16(D), gam,
                                xm.astype(np.float32))


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_layer_tail_bf16(qw, ctx, oracle, relerr, M):
    mats, (wo, gu, dn) = _bf16_case(qw, ctx, oracle, 5100 + M)
    gam = dev(mats[4])
    core = dev(oracle.round_bf16(oracle.normal((M, KO), 5150 + M)), torch.bfloat16)
    x0 = dev(oracle.normal((M, H), 5160 + M))
    x = x0.clone()
    qw.layer_tail(ctx, wo, core, gu, dn, x, gamma=gam)
    z = x0.clone()   # the two calls it replaces
    qw.linear(ctx, wo, core, z, residual=z)
    qw.mlp_fused(ctx, gu, dn, z, z, gamma=gam, residual=z)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    ref = _ref_bf16(oracle, mats, host(core), host(x0))
    assert relerr(host(x), ref) <= 1e-2
    assert relerr(host(x), host(z).astype(np.float64)) <= 1e-3


def test_layer_tail_repeat_and_ld(qw, ctx, oracle, relerr):
    """Consecutive calls with new inputs (the stage's counters must be back at
    zero: a stale count would let the block read the previous x_mid), a core
    with a row stride, and a smaller M on the second call."""
    mats, (wo, gu, dn) = _bf16_case(qw, ctx, oracle, 5200)
    gam = dev(mats[4])
    for it, M in enumerate([4, 2, 1, 3]):
        wide = dev(oracle.round_bf16(oracle.normal((M, KO + 64), 5210 + it)), torch.bfloat16)
        core = wide[:, 32:32 + KO]
        x0 = dev(oracle.normal((M, H), 5220 + it))
        x = x0.clone()
        qw.layer_tail(ctx, wo, core, gu, dn, x, gamma=gam)
        torch.cuda.synchronize()
        assert ctx.device_error() == 0
        ref = _ref_bf16(oracle, mats, host(core), host(x0))
        assert relerr(host(x), ref) <= 1e-2, f"call {it} (M={M})"


@pytest.mark.parametrize("M", [1, 4])
def test_layer_tail_int8(qw, ctx, oracle, relerr, M):
    (qo, so), (qg, sg), (qu, su), (qd, sd) = (
        oracle.quantize_rowscale(oracle.normal(s, 5300 + i, 0.0, 0.02))
        for i, s in enumerate([(H, KO), (I, H), (I, H), (H, I)]))
    gam_h = oracle.normal((H,), 5309, 0.0, 0.05)
    wo = qw.Weight.pack(ctx, qo, qw.WFMT_INT8, scales=so)
    gu = qw.Weight.pack_glu(ctx, qg, qu, qw.WFMT_INT8, gate_scales=sg, up_scales=su)
    dn = qw.Weight.pack(ctx, qd, qw.WFMT_INT8, scales=sd)
    gam = dev(gam_h)
    core = dev(oracle.round_bf16(oracle.normal((M, KO), 5350 + M)), torch.bfloat16)
    x0 = dev(oracle.normal((M, H), 5360 + M))
    x = x0.clone()
    qw.layer_tail(ctx, wo, core, gu, dn, x, gamma=gam)
    z = x0.clone()
    qw.linear(ctx, wo, core, z, residual=z)
    qw.mlp_fused(ctx, gu, dn, z, z, gamma=gam, residual=z)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    f16 = lambda a: a.astype(np.float16).astype(np.float64)
    c = host(core).astype(np.float64)
    xm = host(x0).astype(np.float64) + (c @ qo.astype(np.float64).T) * so
    inv = 1.0 / np.sqrt((xm * xm).mean(axis=1, keepdims=True) + 1e-6)
    b = xm * (1.0 + gam_h.astype(np.float64))[None, :]
    g = (b @ qg.astype(np.float64).T) * sg * inv
    u = (b @ qu.astype(np.float64).T) * su * inv
    h = f16(g / (1.0 + np.exp(-g)) * u)
    ref = xm + (h @ qd.astype(np.float64).T) * sd
    assert relerr(host(x), ref) <= 1e-3
    assert relerr(host(x), host(z).astype(np.float64)) <= 1e-3


def test_layer_tail_fallback_and_graph(qw, ctx, oracle, relerr):
    """M = 6 takes the two-call route; a captured graph of two one-launch
    calls (different weights) replayed 3 times matches the eager calls bit for
    bit, with the inputs reset before every replay."""
    mats, (wo, gu, dn) = _bf16_case(qw, ctx, oracle, 5400)
    gam = dev(mats[4])
    M = 6
    core = dev(oracle.round_bf16(oracle.normal((M, KO), 5450)), torch.bfloat16)
    x0 = dev(oracle.normal((M, H), 5460))
    x = x0.clone()
    qw.layer_tail(ctx, wo, core, gu, dn, x, gamma=gam)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    assert relerr(host(x), _ref_bf16(oracle, mats, host(core), host(x0))) <= 1e-2

    mats2, (wo2, gu2, dn2) = _bf16_case(qw, ctx, oracle, 5500)
    gam2 = dev(mats2[4])
    M = 2
    core = dev(oracle.round_bf16(oracle.normal((M, KO), 5550)), torch.bfloat16)
    x0 = dev(oracle.normal((M, H), 5560))
    x = x0.clone()
    s = torch.cuda.Stream()

    def body():
        qw.layer_tail(ctx, wo, core, gu, dn, x, gamma=gam, stream=s)
        qw.layer_tail(ctx, wo2, core, gu2, dn2, x, gamma=gam2, stream=s)

    with torch.cuda.stream(s):
        body()
    s.synchronize()
    eager = x.clone()
    with torch.cuda.stream(s):
        x.copy_(x0)
        g = qw.Graph(ctx, s)
        with g:
            body()
    for rep in range(3):
        with torch.cuda.stream(s):
            x.copy_(x0)
            g.launch(s)
        s.synchronize()
        assert torch.equal(x, eager), f"replay {rep}"
    assert ctx.device_error() == 0
