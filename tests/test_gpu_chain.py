"""GPU parity of the projection chain (qw_chain_create / qw_chain_launch,
csrc/qw_chain.hip): a decoder's projection sequence over several layers in
one persistent launch at one or two decode tokens.

The chain per layer follows CudaLayer::forward (cuda_engine.cu:105-124):
    in   : x -> [QKV|Z|a|b] or [Q+gate|K|V]         (RMSNorm prologue on some)
    out  : its first 2048 values -> x, + x          (the core's output stand-in)
    gate/up : x -> h (SiLU*mul)                      (RMSNorm prologue on some)
    down : h -> x, + x
The reference is the same sequence on the host: the reference's
dequant-then-matmul for INT8 weights (oracle.linear_int8, mlp_cuda.cu:158-180)
or FP64 products of the BF16 weights, each op's output rounded to the slot's
16-bit type as the chain stores it, and the RMSNorm prologue as the chain
applies it (x * (1 + gamma) rounded to the slot type into the products, 1/rms
on the sums; RMSNorm itself: language_common.cpp:21-36).  The rounding points
match; what differs is the FP32 summation order, through which a stored value
can round the other way (one 16-bit unit) and carry that into the later ops.
Bars: INT8 <= 1e-3 normwise, BF16 <= 1e-2 (the BF16 parity bar: a BF16 unit
is 2^-8 relative, eight times the F16 one).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def _silu(v):
    return v / (1.0 + np.exp(-v))


def _inv_rms(x, eps=1e-6):
    x = np.asarray(x, np.float64)
    return 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def _layers(oracle, fmt, n_layers, seed):
    """Per layer: the stacked input projection, out, gate/up, down (+ gammas)."""
    H, I = 1024, 3584
    layers = []
    for li in range(n_layers):
        n_in = 8192 if li % 2 == 0 else 5120
        shapes = {"in": (n_in, H), "out": (H, 2048), "g": (I, H), "u": (I, H), "down": (H, I)}
        L = {"n_in": n_in}
        for k, (n, kk) in shapes.items():
            sd = seed + 100 * li + len(L)
            if fmt == "int8":
                L[k] = (oracle.int8_uniform((n, kk), sd), oracle.uniform((n,), sd + 1, 2e-5, 2.5e-4))
            else:
                L[k] = oracle.round_bf16(oracle.normal((n, kk), sd, 0.0, 0.02))
        L["gamma_in"] = oracle.normal((H,), seed + 100 * li + 50, 0.0, 0.02) if li == 1 else None
        L["gamma_gu"] = oracle.normal((H,), seed + 100 * li + 51, 0.0, 0.02) if li % 2 == 0 else None
        layers.append(L)
    return layers


def _pack(qw, ctx, fmt, L):
    if fmt == "int8":
        wf = qw.WFMT_INT8
        w = {k: qw.Weight.pack(ctx, L[k][0], wf, scales=L[k][1]) for k in ("in", "out", "down")}
        w["gu"] = qw.Weight.pack_glu(ctx, L["g"][0], L["u"][0], wf, gate_scales=L["g"][1], up_scales=L["u"][1])
    else:
        wf = qw.WFMT_BF16
        w = {k: qw.Weight.pack(ctx, L[k], wf) for k in ("in", "out", "down")}
        w["gu"] = qw.Weight.pack_glu(ctx, L["g"], L["u"], wf)
    return w


def _reference(oracle, fmt, layers, x0):
    rnd = oracle.round_f16 if fmt == "int8" else oracle.round_bf16

    def lin(W, v):
        if fmt == "int8":
            return oracle.linear_int8(W[0], W[1], np.asarray(v, np.float32)).astype(np.float64)
        return np.asarray(v, np.float64) @ W.astype(np.float64).T

    def normed(v, g):
        # the chain's RMSNorm prologue: x * (1 + gamma) rounded to the slot
        # type feeds the MFMA, 1/rms scales the dot products
        xg = rnd((np.asarray(v, np.float64) * (1.0 + np.asarray(g, np.float64))).astype(np.float32))
        return xg, _inv_rms(v)

    x = np.asarray(x0, np.float64)
    bigs = []
    for L in layers:
        if L["gamma_in"] is not None:
            xg, inv = normed(x, L["gamma_in"])
            pre = lin(L["in"], xg) * inv
        else:
            pre = lin(L["in"], x)
        big = rnd(pre.astype(np.float32)).astype(np.float64)
        bigs.append(big)
        x = rnd((lin(L["out"], big[:, :2048]) + x).astype(np.float32)).astype(np.float64)
        if L["gamma_gu"] is not None:
            xg, inv = normed(x, L["gamma_gu"])
            g, u = lin(L["g"], xg) * inv, lin(L["u"], xg) * inv
        else:
            g, u = lin(L["g"], x), lin(L["u"], x)
        h = rnd((_silu(g) * u).astype(np.float32)).astype(np.float64)
        x = rnd((lin(L["down"], h) + x).astype(np.float32)).astype(np.float64)
    return x, bigs


def _build(qw, ctx, fmt, layers, ws, xt, xout, bigout, M):
    """Slots: 0 = x (imported from xt, exported to xout), 1 = big (exported),
    2 = h."""
    code = qw.F16 if fmt == "int8" else qw.BF16
    slots = [{"len": 1024, "init": xt, "out": xout}, {"len": 8192, "out": bigout}, {"len": 3584}]
    ops = []
    for L, w in zip(layers, ws):
        gi = None if L["gamma_in"] is None else dev(L["gamma_in"])
        gg = None if L["gamma_gu"] is None else dev(L["gamma_gu"])
        ops.append({"w": w["in"], "in": 0, "out": 1, "gamma": gi})
        ops.append({"w": w["out"], "in": 1, "out": 0, "residual": True})
        ops.append({"w": w["gu"], "in": 0, "out": 2, "gamma": gg})
        ops.append({"w": w["down"], "in": 2, "out": 0, "residual": True})
    return qw.Chain(ctx, code, M, slots, ops)


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("fmt", ["int8", "bf16"])
def test_chain_layers(qw, ctx, oracle, relerr, fmt, M):
    n_layers = 3
    layers = _layers(oracle, fmt, n_layers, 4000 + M)
    ws = [_pack(qw, ctx, fmt, L) for L in layers]
    dt = torch.float16 if fmt == "int8" else torch.bfloat16
    x0 = oracle.normal((M, 1024), 4090 + M)
    xt = dev(x0, dt)
    xout = torch.zeros(M, 1024, device="cuda", dtype=dt)
    bigout = torch.zeros(M, 8192, device="cuda", dtype=dt)
    ch = _build(qw, ctx, fmt, layers, ws, xt, xout, bigout, M)
    ch.launch()
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    ref_x, bigs = _reference(oracle, fmt, layers, host(xt))
    bar = 1e-3 if fmt == "int8" else 1e-2
    assert relerr(host(xout), ref_x) <= bar
    n_last = layers[-1]["n_in"]
    assert relerr(host(bigout)[:, :n_last], bigs[-1]) <= bar
    # replays: bit-identical (new epoch each launch, no state carried over)
    first = xout.clone()
    for _ in range(4):
        xout.zero_()
        ch.launch()
        torch.cuda.synchronize()
        assert torch.equal(xout, first)
    ch.close()


def test_chain_graph_replay(qw, ctx, oracle):
    """Captured in a graph and replayed with new inputs in between: every
    replay equals an eager launch on the same input."""
    fmt, M = "int8", 1
    layers = _layers(oracle, fmt, 2, 4200)
    ws = [_pack(qw, ctx, fmt, L) for L in layers]
    xt = dev(oracle.normal((M, 1024), 4201), torch.float16)
    xout = torch.zeros(M, 1024, device="cuda", dtype=torch.float16)
    bigout = torch.zeros(M, 8192, device="cuda", dtype=torch.float16)
    ch = _build(qw, ctx, fmt, layers, ws, xt, xout, bigout, M)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        g = qw.Graph(ctx, stream)
        with g:
            ch.launch(stream)
        for rep in range(3):
            xt.copy_(dev(oracle.normal((M, 1024), 4210 + rep), torch.float16))
            g.launch(stream)
            stream.synchronize()
            got = xout.clone()
            ch.launch(stream)
            stream.synchronize()
            assert torch.equal(got, xout)
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    ch.close()


def test_chain_rejects_bad_plans(qw, ctx, oracle):
    """The host refuses chains the kernel cannot run safely."""
    layers = _layers(oracle, "int8", 1, 4300)
    w = _pack(qw, ctx, "int8", layers[0])
    xt = torch.zeros(1, 1024, device="cuda", dtype=torch.float16)
    slots = [{"len": 1024, "init": xt}, {"len": 8192}, {"len": 3584}]
    bad = [
        # op 1 does not read op 0's output
        [{"w": w["in"], "in": 0, "out": 1}, {"w": w["gu"], "in": 0, "out": 2}],
        # input slot never written
        [{"w": w["down"], "in": 2, "out": 0}],
        # reads its own output slot
        [{"w": w["gu"], "in": 0, "out": 0}],
        # residual rows never written
        [{"w": w["in"], "in": 0, "out": 1, "residual": True}],
        # input range beyond the rows written
        [{"w": w["in"], "in": 0, "out": 1}, {"w": w["out"], "in": 1, "out": 0, "in_offset": 7168}],
    ]
    for ops in bad:
        with pytest.raises(qw.QwError):
            qw.Chain(ctx, qw.F16, 1, slots, ops)
    with pytest.raises(qw.QwError):  # BF16 slots for INT8 weights
        qw.Chain(ctx, qw.BF16, 1, slots, [{"w": w["in"], "in": 0, "out": 1}])


def test_chain_epoch_wrap(qw, ctx, oracle):
    """The tag keeps 22 bits of the launch epoch.  Launches run across the
    wrap (epoch set just below it through the test hook): the epoch skips the
    field value 0, the launch at which the field returns to 1 clears every
    slot word behind a grid barrier, and every launch equals the first one."""
    fmt, M = "int8", 2
    layers = _layers(oracle, fmt, 2, 4400)
    ws = [_pack(qw, ctx, fmt, L) for L in layers]
    xt = dev(oracle.normal((M, 1024), 4401), torch.float16)
    xout = torch.zeros(M, 1024, device="cuda", dtype=torch.float16)
    bigout = torch.zeros(M, 8192, device="cuda", dtype=torch.float16)
    ch = _build(qw, ctx, fmt, layers, ws, xt, xout, bigout, M)
    ch.launch()
    torch.cuda.synchronize()
    first = xout.clone()
    wrap = 1 << 22
    ch.epoch(set_to=wrap - 2)
    seen = []
    for _ in range(4):
        xout.zero_()
        seen.append(ch.epoch())
        ch.launch()
        torch.cuda.synchronize()
        assert torch.equal(xout, first)
    seen.append(ch.epoch())
    # wrap - 2, wrap - 1, (wrap skipped: field 0) wrap + 1 = the clearing launch, wrap + 2, ...
    assert seen == [wrap - 2, wrap - 1, wrap + 1, wrap + 2, wrap + 3]
    with pytest.raises(qw.QwError):
        ch.epoch(set_to=wrap)
    assert ctx.device_error() == 0
    ch.close()
