"""GPU parity of qw_mlp_stack (L consecutive MLP blocks; at decode one
persistent launch) against L calls of qw_mlp_fused and against the oracle's
FP64 block composition.

Bars: BF16 weights, one block: <= 1e-2 normwise vs FP64 on the BF16-rounded
weights; L blocks with x rounded to BF16 after every block: every block
<= 1e-2 against FP64 on its own input (teacher forcing), and end to end
<= 1e-2 + 2 e_ref vs the FP64 composition, e_ref being the distance of the
reference's own BF16 chain (BF16-in / BF16-out GEMVs) on the same inputs
(test_mlp_stack_bench_configs states why); vs L qw_mlp_fused calls <= 1e-2
(the same math with the gate/up K slices summed in another grouping, which
moves a BF16 rounding of the hidden state now and then).  INT8 weights
<= 1e-3 vs the dequant-then-matmul composition on the same q, s and F16
roundings.  Every launch must leave the device error
flag clear.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

H, I = 1024, 3584


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def _layers(oracle, L, seed):
    out = []
    for l in range(L):
        G = oracle.normal((I, H), seed + 10 * l, 0.0, 0.02)
        U = oracle.normal((I, H), seed + 10 * l + 1, 0.0, 0.02)
        D = oracle.normal((H, I), seed + 10 * l + 2, 0.0, 0.02)
        gam = oracle.normal((H,), seed + 10 * l + 3, 0.0, 0.05)
        out.append((G, U, D, gam))
    return out


def _ref_bf16(oracle, layers, x):
    """FP64 blocks on the BF16-rounded weights, x rounded to BF16 after each."""
    x = x.astype(np.float64)
    for G, U, D, gam in layers:
        y = oracle.mlp_block_f64(oracle.round_bf16(G), oracle.round_bf16(U), oracle.round_bf16(D), gam,
                                 x.astype(np.float32))
        x = oracle.round_bf16(y.astype(np.float32)).astype(np.float64)
    return x


def _ref_bf16_block(oracle, G, U, D, gam, x):
    """One MLP block as the reference's BF16 path computes it: every GEMV a
    cublasGemmEx with BF16 operands and BF16 output, FP32 accumulation
    (bf16_gemv / bf16_gemv_add, bf16_gemm.cuh:82-120): the normalized input,
    gate, up, h and the new hidden state each rounded to BF16."""
    x = np.asarray(x, np.float32)
    inv = (1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)).astype(np.float32)
    xn = oracle.round_bf16(x * inv * (1.0 + np.asarray(gam, np.float32))[None, :])
    g = oracle.round_bf16(xn @ G.T)
    u = oracle.round_bf16(xn @ U.T)
    h = oracle.round_bf16((g / (1.0 + np.exp(-g)) * u).astype(np.float32))
    return oracle.round_bf16((h @ D.T + x).astype(np.float32))


def _chain_bar(oracle, layers, x, ref64):
    """The multi-block BF16 bar: 1e-2 + 2 e_ref, e_ref = the distance from the
    FP64 composition `ref64` of the reference's own BF16 chain on the same
    inputs (_ref_bf16_block composed over the layers); see
    test_mlp_stack_bench_configs for why."""
    x = np.asarray(x, np.float32)
    for G, U, D, gam in layers:
        x = _ref_bf16_block(oracle, oracle.round_bf16(G), oracle.round_bf16(U), oracle.round_bf16(D), gam, x)
    den = np.abs(ref64).max()
    return 1e-2 + 2.0 * float(np.abs(x - ref64).max() / den)


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("L", [1, 5])
def test_mlp_stack_bf16(qw, ctx, oracle, relerr, M, L):
    layers = _layers(oracle, L, 2100 + L)
    gu = [qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16) for G, U, _, _ in layers]
    dn = [qw.Weight.pack(ctx, D, qw.WFMT_BF16) for _, _, D, _ in layers]
    gms = [dev(gam) for *_, gam in layers]
    x0 = dev(oracle.normal((M, H), 2199 + M), torch.bfloat16)
    y = torch.empty_like(x0)
    qw.mlp_stack(ctx, gu, dn, x0, y, gammas=gms)
    # the same blocks as L separate qw_mlp_fused calls
    z = x0.clone()
    for l in range(L):
        qw.mlp_fused(ctx, gu[l], dn[l], z, z, gamma=gms[l], residual=z)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    ref = _ref_bf16(oracle, layers, host(x0))
    # the multi-block bar (1e-2 for one block)
    e_stack, e_blocks = relerr(host(y), ref), relerr(host(z), ref)
    bar = _chain_bar(oracle, layers, host(x0), ref)
    print("first launch rel err: stack", e_stack, "per-block", e_blocks, "bar", bar)
    assert e_stack <= bar and e_blocks <= bar
    # same math as the per-block launches; the K slices of the gate/up
    # reduction are summed in another grouping, which moves a BF16 rounding of
    # the hidden state now and then
    assert relerr(host(y), host(z).astype(np.float64)) <= 1e-2
    # a second launch on other inputs (new epoch tags), in place
    x1 = dev(oracle.normal((M, H), 2299 + M), torch.bfloat16)
    x1h = host(x1)
    r1 = _ref_bf16(oracle, layers, x1h)
    z1 = x1.clone()
    qw.mlp_stack(ctx, gu, dn, x1, x1, gammas=gms)
    for l in range(L):
        qw.mlp_fused(ctx, gu[l], dn[l], z1, z1, gamma=gms[l], residual=z1)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    e_stack, e_blocks = relerr(host(x1), r1), relerr(host(z1), r1)
    bar = _chain_bar(oracle, layers, x1h, r1)
    print("second launch rel err: stack", e_stack, "per-block", e_blocks, "bar", bar)
    assert e_stack <= bar and e_blocks <= bar
    assert relerr(host(x1), host(z1).astype(np.float64)) <= 1e-2


def test_mlp_stack_bf16_folded_norm_24_layers(qw, ctx, oracle, relerr):
    """24 blocks, the norm weights folded into the gate/up weights."""
    L, M = 24, 1
    layers = _layers(oracle, L, 2400)
    gu, dn = [], []
    for G, U, D, gam in layers:
        w = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16)
        w.fold_norm(dev(gam))
        gu.append(w)
        dn.append(qw.Weight.pack(ctx, D, qw.WFMT_BF16))
    x0 = dev(oracle.normal((M, H), 2499), torch.bfloat16)
    y = torch.empty_like(x0)
    qw.mlp_stack(ctx, gu, dn, x0, y)
    z = x0.clone()
    for l in range(L):
        qw.mlp_fused(ctx, gu[l], dn[l], z, z, residual=z)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    # folding rounds W*(1+gamma) to BF16: compare with the folded weights
    x = host(x0).astype(np.float64)
    for G, U, D, gam in layers:
        Gf = oracle.round_bf16(oracle.round_bf16(G) * (1.0 + gam)[None, :].astype(np.float32))
        Uf = oracle.round_bf16(oracle.round_bf16(U) * (1.0 + gam)[None, :].astype(np.float32))
        yb = oracle.mlp_block_f64(Gf, Uf, oracle.round_bf16(D), np.zeros(H, np.float32), x.astype(np.float32))
        x = oracle.round_bf16(yb.astype(np.float32)).astype(np.float64)
    # the multi-block bar, on the folded weights
    xf = host(x0)
    for G, U, D, gam in layers:
        Gf = oracle.round_bf16(oracle.round_bf16(G) * (1.0 + gam)[None, :].astype(np.float32))
        Uf = oracle.round_bf16(oracle.round_bf16(U) * (1.0 + gam)[None, :].astype(np.float32))
        xf = _ref_bf16_block(oracle, Gf, Uf, oracle.round_bf16(D), np.zeros(H, np.float32), xf)
    bar = 1e-2 + 2.0 * relerr(xf, x)
    e_stack, e_blocks = relerr(host(y), x), relerr(host(z), x)
    print("24-layer rel err: stack", e_stack, "per-block", e_blocks, "bar", bar)
    assert e_stack <= bar and e_blocks <= bar


@pytest.mark.parametrize("M", [1, 2, 3, 4, 8])
def test_mlp_stack_int8(qw, ctx, oracle, relerr, M):
    """INT8 weights (per-row scales), F16 x; the reference composition is the
    dequant-then-matmul of the same q and s (in FP64) with the kernel's F16
    roundings of x * (1 + gamma), h and the hidden state."""
    L = 3
    layers = []
    for l in range(L):
        # N(0, 0.02) weights quantized by the reference recipe (per-row scales
        # ~6e-4): hidden states stay in the F16 range over the blocks
        (qg, sg), (qu, su), (qd, sd) = (oracle.quantize_rowscale(oracle.normal(s, 2600 + 10 * l + i, 0.0, 0.02))
                                        for i, s in enumerate([(I, H), (I, H), (H, I)]))
        gam = oracle.normal((H,), 2608 + 10 * l, 0.0, 0.05)
        layers.append((qg, qu, qd, sg, su, sd, gam))
    gu = [qw.Weight.pack_glu(ctx, qg, qu, qw.WFMT_INT8, gate_scales=sg, up_scales=su)
          for qg, qu, _, sg, su, _, _ in layers]
    dn = [qw.Weight.pack(ctx, qd, qw.WFMT_INT8, scales=sd) for _, _, qd, _, _, sd, _ in layers]
    gms = [dev(L_[6]) for L_ in layers]
    x0 = dev(oracle.normal((M, H), 2699), torch.float16)
    y = torch.empty_like(x0)
    qw.mlp_stack(ctx, gu, dn, x0, y, gammas=gms)
    z = x0.clone()
    for l in range(L):   # the two-launch INT8 MLP path (qw_mlp_fused's default for INT8)
        qw.mlp_fused(ctx, gu[l], dn[l], z, z, gamma=gms[l], residual=z)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    x = host(x0).astype(np.float64)
    f16 = lambda a: a.astype(np.float16).astype(np.float64)
    for qg, qu, qd, sg, su, sd, gam in layers:
        inv = 1.0 / np.sqrt((x * x).mean(axis=1, keepdims=True) + 1e-6)
        b = f16(x * (1.0 + gam.astype(np.float64))[None, :])    # the F16 MFMA input
        g = (b @ qg.astype(np.float64).T) * sg * inv
        u = (b @ qu.astype(np.float64).T) * su * inv
        h = f16(g / (1.0 + np.exp(-g)) * u)
        x = f16(x + (h @ qd.astype(np.float64).T) * sd)
    assert relerr(host(y), x) <= 1e-3
    assert relerr(host(y), host(z).astype(np.float64)) <= 1e-3


@pytest.mark.parametrize("M", [1, 8])
def test_mlp_stack_int8_bench_config(qw, ctx, oracle, relerr, M):
    """The INT8 configuration bench.py times on the persistent stack
    (cfg3_int8_mlp_stack_M1 / _M8): 24 INT8 blocks with per-row scales and a
    per-call gamma, F16 x, one launch.  Teacher-forced per-block bar: the
    launch of the first n blocks against the FP64 block n (dequant-then-
    matmul of the same q and s, with the kernel's F16 roundings of
    x * (1 + gamma), h and the hidden state) on the output of the first
    n - 1: <= 1e-3, the INT8 bar; the full launch equals the last prefix."""
    L = 24
    layers = []
    for l in range(L):
        (qg, sg), (qu, su), (qd, sd) = (oracle.quantize_rowscale(oracle.normal(s, 4600 + 10 * l + i, 0.0, 0.02))
                                        for i, s in enumerate([(I, H), (I, H), (H, I)]))
        gam = oracle.normal((H,), 4608 + 10 * l, 0.0, 0.02)
        layers.append((qg, qu, qd, sg, su, sd, gam))
    gu = [qw.Weight.pack_glu(ctx, qg, qu, qw.WFMT_INT8, gate_scales=sg, up_scales=su)
          for qg, qu, _, sg, su, _, _ in layers]
    dn = [qw.Weight.pack(ctx, qd, qw.WFMT_INT8, scales=sd) for _, _, qd, _, _, sd, _ in layers]
    gms = [dev(L_[6]) for L_ in layers]
    x0 = dev(oracle.normal((M, H), 4699 + M), torch.float16)
    f16 = lambda a: a.astype(np.float16).astype(np.float64)
    prev = host(x0).astype(np.float64)
    last = None
    for n in range(1, L + 1):
        y = torch.empty_like(x0)
        qw.mlp_stack(ctx, gu[:n], dn[:n], x0, y, gammas=gms[:n])
        torch.cuda.synchronize()
        got = host(y).astype(np.float64)
        qg, qu, qd, sg, su, sd, gam = layers[n - 1]
        inv = 1.0 / np.sqrt((prev * prev).mean(axis=1, keepdims=True) + 1e-6)
        b = f16(prev * (1.0 + gam.astype(np.float64))[None, :])
        g = (b @ qg.astype(np.float64).T) * sg * inv
        u = (b @ qu.astype(np.float64).T) * su * inv
        h = f16(g / (1.0 + np.exp(-g)) * u)
        ref = f16(prev + (h @ qd.astype(np.float64).T) * sd)
        e = relerr(got, ref)
        assert e <= 1e-3, f"block {n}: {e}"
        prev = got
        last = y
    assert ctx.device_error() == 0
    # the graph-replayed form the bench times gives the same bits
    z = torch.empty_like(x0)
    s_ = torch.cuda.Stream()
    with torch.cuda.stream(s_):
        g_ = qw.Graph(ctx, s_)
        with g_:
            qw.mlp_stack(ctx, gu, dn, x0, z, gammas=gms, stream=s_)
        for _ in range(3):
            g_.launch(s_)
    s_.synchronize()
    assert torch.equal(z, last)
    assert ctx.device_error() == 0


def test_mlp_stack_graph_replays(qw, ctx, oracle, relerr):
    """Captured once, replayed three times with eager work between: every
    replay (a new epoch each) equals the eager result."""
    L, M = 4, 1
    layers = _layers(oracle, L, 2800)
    gu = [qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16) for G, U, _, _ in layers]
    dn = [qw.Weight.pack(ctx, D, qw.WFMT_BF16) for _, _, D, _ in layers]
    gms = [dev(gam) for *_, gam in layers]
    x0 = dev(oracle.normal((M, H), 2899), torch.bfloat16)
    buf = torch.empty_like(x0)
    eager = torch.empty_like(x0)
    qw.mlp_stack(ctx, gu, dn, x0, eager, gammas=gms)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    g = qw.Graph(ctx, stream)
    with torch.cuda.stream(stream):
        buf.copy_(x0)
        stream.synchronize()
        with g:
            qw.mlp_stack(ctx, gu, dn, buf, buf, gammas=gms, stream=stream)
    for _ in range(3):
        buf.copy_(x0)
        torch.cuda.synchronize()
        g.launch(stream)
        stream.synchronize()
        assert torch.equal(buf, eager)
        other = torch.empty_like(x0)
        qw.mlp_fused(ctx, gu[0], dn[0], x0, other, gamma=gms[0], residual=x0)  # eager work between replays
        torch.cuda.synchronize()
    assert ctx.device_error() == 0


def test_mlp_stack_fallback_more_tokens(qw, ctx, oracle, relerr):
    """M = 9 takes the per-block launches: identical to qw_mlp_fused calls."""
    L, M = 2, 9
    layers = _layers(oracle, L, 2900)
    gu = [qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16) for G, U, _, _ in layers]
    dn = [qw.Weight.pack(ctx, D, qw.WFMT_BF16) for _, _, D, _ in layers]
    gms = [dev(gam) for *_, gam in layers]
    x0 = dev(oracle.normal((M, H), 2999), torch.bfloat16)
    y = torch.empty_like(x0)
    qw.mlp_stack(ctx, gu, dn, x0, y, gammas=gms)
    z = x0.clone()
    for l in range(L):
        qw.mlp_fused(ctx, gu[l], dn[l], z, z, gamma=gms[l], residual=z)
    torch.cuda.synchronize()
    assert torch.equal(y, z)


def test_mlp_stack_epoch_wrap_varying_m(qw, ctx, oracle):
    """The tag keeps 26 bits of the launch epoch.  A launch with 8 tokens
    leaves words of tokens 1..7 behind; launches with 1 token then run up to
    the wrap (epoch set just below it through the test hook), where the
    launch whose field is 0 clears every word behind a grid barrier; an
    8-token launch at the first launch's field value then equals the same
    launch at a fresh epoch (stale words would have matched its tags)."""
    L = 3
    layers = _layers(oracle, L, 3100)
    gu = [qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16) for G, U, _, _ in layers]
    dn = [qw.Weight.pack(ctx, D, qw.WFMT_BF16) for _, _, D, _ in layers]
    gms = [dev(gam) for *_, gam in layers]
    xa = dev(oracle.normal((8, H), 3190), torch.bfloat16)
    xb = dev(oracle.normal((8, H), 3191), torch.bfloat16)
    x1 = dev(oracle.normal((1, H), 3192), torch.bfloat16)

    def run(x):
        y = torch.empty_like(x)
        qw.mlp_stack(ctx, gu, dn, x, y, gammas=gms)
        torch.cuda.synchronize()
        return y

    ref_b, ref_1 = run(xb), run(x1)
    f = 1 << 26
    ctx.stack_epoch(set_to=2 * f + 5)
    run(xa)                               # field 5: tokens 0..7, both parities
    ctx.stack_epoch(set_to=3 * f - 2)
    seen = []
    for _ in range(3):                    # fields f-2, f-1 and 0 (the clearing launch)
        seen.append(ctx.stack_epoch())
        assert torch.equal(run(x1), ref_1)
    assert seen == [3 * f - 2, 3 * f - 1, 3 * f]
    assert ctx.stack_epoch() == 3 * f + 1
    ctx.stack_epoch(set_to=3 * f + 5)     # field 5 again, as the 8-token launch above
    assert torch.equal(run(xb), ref_b)
    assert ctx.device_error() == 0


_BENCH_LAYERS = {}


def _bench_layers(oracle):
    """24 layers shaped as bench.py's: BF16-rounded N(0, 0.02) weights, a
    per-layer RMSNorm weight N(0, 0.02) (the norm scales by 1 + w)."""
    if not _BENCH_LAYERS:
        out = []
        for l in range(24):
            G, U, D = (oracle.round_bf16(oracle.normal(s, 3300 + 10 * l + i, 0.0, 0.02))
                       for i, s in enumerate([(I, H), (I, H), (H, I)]))
            out.append((G, U, D, oracle.normal((H,), 3303 + 10 * l, 0.0, 0.02)))
        _BENCH_LAYERS["v"] = out
    return _BENCH_LAYERS["v"]


@pytest.mark.parametrize("route", ["headline_M1_gamma", "cfg2_M8_folded"])
def test_mlp_stack_bench_configs(qw, ctx, oracle, relerr, route):
    """The two configurations bench.py times on the persistent stack, exactly:
    24 BF16 blocks in one launch replayed from a graph in place, M = 1 with a
    per-call gamma (the headline) and M = 8 with gamma folded into gate/up
    (configs[1] at M = 8).

    Bars (the multi-block bar of the parity contract):
      * every block, against FP64 of that block on the kernel's own BF16 input
        (teacher forcing): <= 1e-2, the per-call BF16 bar.  The input of
        block l is the output of the launch of the first l - 1 blocks: a
        block's arithmetic does not depend on L, so prefixes are bit-identical
        to the 24-block launch's intermediate states (checked at the end);
      * end to end, against the FP64 composition with the hidden state rounded
        to BF16 after every block: <= 1e-2 + 2 e_ref, where e_ref is how far the
        reference's own BF16 chain (every GEMV a BF16-in / BF16-out GemmEx with
        FP32 accumulation, bf16_gemm.cuh:82-120, composed over the same blocks,
        _ref_bf16_block) lands from that FP64 composition on the same inputs.
        Once a summation-order difference flips one BF16 rounding of the
        hidden state, the residual path carries that unit to the end, so no
        FP32-accumulating chain reproduces the FP64 one closer than such flips
        add up to; the kernel's flips are independent of the reference's, so
        its distance may be up to twice e_ref, plus the one-block bar."""
    M, folded = (1, False) if route == "headline_M1_gamma" else (8, True)
    layers = _bench_layers(oracle)
    L = len(layers)
    gu, dn, gms, ref_w = [], [], [], []
    for G, U, D, gam in layers:
        w = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16)
        if folded:
            w.fold_norm(dev(gam))
            fold = (1.0 + gam)[None, :].astype(np.float32)
            ref_w.append((oracle.round_bf16(G * fold), oracle.round_bf16(U * fold), D, np.zeros(H, np.float32)))
        else:
            gms.append(dev(gam))
            ref_w.append((G, U, D, gam))
        gu.append(w)
        dn.append(qw.Weight.pack(ctx, D, qw.WFMT_BF16))
    x0 = dev(oracle.normal((M, H), 3399 + M), torch.bfloat16)

    def stack(n, x, y, stream=None):
        qw.mlp_stack(ctx, gu[:n], dn[:n], x, y, gammas=(gms[:n] if gms else None), stream=stream)

    # teacher-forced per-block bar on every block
    prev = host(x0)
    ys = []
    for n in range(1, L + 1):
        y = torch.empty_like(x0)
        stack(n, x0, y)
        torch.cuda.synchronize()
        ys.append(host(y))
        G, U, D, gam = ref_w[n - 1]
        e = relerr(ys[-1], oracle.mlp_block_f64(G, U, D, gam, prev))
        assert e <= 1e-2, f"block {n}: {e}"
        prev = ys[-1]
    assert ctx.device_error() == 0

    # the bench form: the 24-block launch captured once, replayed in place
    buf = x0.clone()
    stream = torch.cuda.Stream()
    g = qw.Graph(ctx, stream)
    with torch.cuda.stream(stream):
        stream.synchronize()
        with g:
            stack(L, buf, buf, stream=stream)
    for _ in range(3):
        buf.copy_(x0)
        torch.cuda.synchronize()
        g.launch(stream)
        stream.synchronize()
        assert np.array_equal(host(buf), ys[-1])
    assert ctx.device_error() == 0

    # end-to-end bar against the FP64 composition
    x64 = host(x0).astype(np.float64)
    xr = host(x0)
    for G, U, D, gam in ref_w:
        x64 = oracle.round_bf16(oracle.mlp_block_f64(G, U, D, gam, x64.astype(np.float32)).astype(np.float32))
        x64 = x64.astype(np.float64)
        xr = _ref_bf16_block(oracle, G, U, D, gam, xr)
    e_ref = relerr(xr, x64)
    e = relerr(ys[-1], x64)
    print(f"{route}: 24-block rel err {e:.3e}; reference BF16 chain {e_ref:.3e}")
    assert e <= 1e-2 + 2.0 * e_ref
