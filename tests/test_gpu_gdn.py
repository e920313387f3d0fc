"""GPU parity of the Gated-DeltaNet decode step (qw_gdn_decode) against the
CPU oracle (orc_gdn_step, pinned bit-exactly to the reference's own
LinearAttention::forward in tests/test_oracle.py).

Shapes: Qwen3.5-0.8B linear attention, 16 heads, key_dim = value_dim = 128,
conv kernel 4 (also 1 and 2).  Several consecutive tokens run on the GPU
with the states carried in place, and on the oracle with its own states.

Bars: FP32 outputs and states <= 1e-5 normwise against the oracle (only the
summation order of the column dot products and norms differs; the carried
state accumulates that over the steps); the conv state is a pure copy, so it
must match bit for bit; BF16 inputs/outputs: the oracle runs on the same
rounded inputs and the output carries one BF16 rounding (<= 4e-3).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

NH, KD, VD = 16, 128, 128
CD = 2 * NH * KD + NH * VD


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def _params(oracle, K, seed):
    return dict(conv_w=oracle.normal((CD, K), seed, 0.0, 0.5), A_log=oracle.normal((NH,), seed + 1, 0.0, 0.5),
                dt_bias=oracle.normal((NH,), seed + 2, 0.0, 0.5),
                norm_w=1.0 + oracle.normal((VD,), seed + 3, 0.0, 0.1))


@pytest.mark.parametrize("B,K,io", [(1, 4, "f32"), (3, 4, "f32"), (2, 1, "f32"), (2, 2, "f32"), (4, 4, "bf16")])
def test_gdn_decode_parity(qw, ctx, oracle, relerr, B, K, io):
    P = _params(oracle, K, 900 + K)
    dP = {k: dev(v) for k, v in P.items()}
    cs = oracle.normal((B, CD, max(K - 1, 0)), 910)
    rs = oracle.normal((B, NH, KD * VD), 911, 0.0, 0.3)
    dcs, drs = dev(cs), dev(rs)
    tdt = torch.float32 if io == "f32" else torch.bfloat16
    # one stacked projection output row per sequence: [mixed | z | a | b | pad]
    ld = CD + NH * VD + 2 * NH + 8
    for step in range(4):
        row = oracle.normal((B, ld), 920 + step)
        drow = dev(row, tdt)
        mixed, z = drow[:, :CD], drow[:, CD:CD + NH * VD]
        a, b = drow[:, CD + NH * VD:CD + NH * VD + NH], drow[:, CD + NH * VD + NH:CD + NH * VD + 2 * NH]
        out = torch.empty(B, NH * VD, device="cuda", dtype=tdt)
        qw.gdn_decode(ctx, dP["conv_w"], dP["A_log"], dP["dt_bias"], dP["norm_w"], mixed, z, a, b, dcs, drs, out,
                      NH)
        torch.cuda.synchronize()
        r = host(drow)
        o_ref, cs, rs = oracle.gdn_step(r[:, :CD], r[:, CD + NH * VD:CD + NH * VD + NH],
                                        r[:, CD + NH * VD + NH:CD + NH * VD + 2 * NH], r[:, CD:CD + NH * VD],
                                        P["conv_w"], P["A_log"], P["dt_bias"], P["norm_w"], cs, rs, NH, KD, VD)
        bar = 1e-5 if io == "f32" else 4e-3
        assert relerr(host(out), o_ref) <= bar, (step, relerr(host(out), o_ref))
        assert relerr(host(drs), rs) <= 1e-5, (step, relerr(host(drs), rs))
        assert np.array_equal(host(dcs), cs)


def test_gdn_decode_repeatable(qw, ctx, oracle):
    """Fixed reduction orders: the same inputs and states give the same bits."""
    B, K = 2, 4
    P = {k: dev(v) for k, v in _params(oracle, K, 930).items()}
    cs0 = dev(oracle.normal((B, CD, K - 1), 931))
    rs0 = dev(oracle.normal((B, NH, KD * VD), 932, 0.0, 0.3))
    row = dev(oracle.normal((B, CD + NH * VD + 2 * NH), 933))
    outs, states = [], []
    for _ in range(3):
        cs, rs = cs0.clone(), rs0.clone()
        out = torch.empty(B, NH * VD, device="cuda")
        qw.gdn_decode(ctx, P["conv_w"], P["A_log"], P["dt_bias"], P["norm_w"], row[:, :CD],
                      row[:, CD:CD + NH * VD], row[:, CD + NH * VD:CD + NH * VD + NH],
                      row[:, CD + NH * VD + NH:], cs, rs, out, NH)
        outs.append(out)
        states.append(rs)
    torch.cuda.synchronize()
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    assert all(torch.equal(states[0], s) for s in states[1:])


def test_gdn_decode_errors(qw, ctx):
    """Shapes the kernel does not cover are refused with a status, not run."""
    P = {"conv_w": torch.zeros(2 * 4 * 64 + 4 * 64, 4, device="cuda"), "A_log": torch.zeros(4, device="cuda"),
         "dt_bias": torch.zeros(4, device="cuda"), "norm_w": torch.ones(64, device="cuda")}
    x = torch.zeros(1, 2048, device="cuda")
    cs = torch.zeros(1, 768 * 3, device="cuda")
    rs = torch.zeros(1, 4 * 64 * 64, device="cuda")
    out = torch.empty(1, 256, device="cuda")
    with pytest.raises(qw.QwError):
        qw.gdn_decode(ctx, P["conv_w"], P["A_log"], P["dt_bias"], P["norm_w"], x, x, x, x, cs, rs, out,
                      4, key_dim=64, value_dim=64)


def _ctx_with(qw, env, **kw):
    import os
    os.environ.update(env)
    try:
        return qw.Context(0, **kw)
    finally:
        for k in env:
            del os.environ[k]


@pytest.fixture(scope="module")
def serial_ctx(qw):
    """Every token run through the one-launch serial kernel."""
    c = _ctx_with(qw, {"QW_GDN_CHUNK_MIN": "1000000000"})
    yield c
    torch.cuda.synchronize()
    c.close()


@pytest.fixture(scope="module")
def chunk_ctx(qw):
    """Every token run (T >= 1) through the chunked form."""
    c = _ctx_with(qw, {"QW_GDN_CHUNK_MIN": "1"})
    yield c
    torch.cuda.synchronize()
    c.close()


@pytest.fixture(scope="module")
def small_ws_ctx(qw):
    """Chunked form with a workspace of ~6 MB beyond the fixed regions: one
    sequence runs in segments of 128 tokens (states carried between the
    segments' launches)."""
    c = _ctx_with(qw, {"QW_GDN_CHUNK_MIN": "1"},
                  workspace_bytes=qw.lib().qw_workspace_query(1, 1, 1) + (6 << 20))
    yield c
    torch.cuda.synchronize()
    c.close()


def _prefill_case(qw, c, oracle, B, T, K, io, seed):
    P = _params(oracle, K, seed)
    dP = {k: dev(v) for k, v in P.items()}
    cs = oracle.normal((B, CD, max(K - 1, 0)), seed + 1)
    rs = oracle.normal((B, NH, KD * VD), seed + 2, 0.0, 0.3)
    dcs, drs = dev(cs), dev(rs)
    tdt = torch.float32 if io == "f32" else torch.bfloat16
    ld = CD + NH * VD + 2 * NH
    rows = dev(oracle.normal((B * T, ld), seed + 3), tdt)
    out = torch.empty(B * T, NH * VD, device="cuda", dtype=tdt)
    qw.gdn_prefill(c, dP["conv_w"], dP["A_log"], dP["dt_bias"], dP["norm_w"], rows[:, :CD],
                   rows[:, CD:CD + NH * VD], rows[:, CD + NH * VD:CD + NH * VD + NH], rows[:, CD + NH * VD + NH:],
                   dcs, drs, out, NH, T)
    torch.cuda.synchronize()
    r = host(rows).reshape(B, T, ld)
    o_ref = np.empty((B, T, NH * VD), np.float32)
    for t in range(T):
        rt = np.ascontiguousarray(r[:, t])
        o_ref[:, t], cs, rs = oracle.gdn_step(rt[:, :CD], rt[:, CD + NH * VD:CD + NH * VD + NH],
                                              rt[:, CD + NH * VD + NH:], rt[:, CD:CD + NH * VD], P["conv_w"],
                                              P["A_log"], P["dt_bias"], P["norm_w"], cs, rs, NH, KD, VD)
    return host(out).reshape(B, T, -1), o_ref, host(drs), rs, host(dcs), cs


# Bars for the chunked form (FP32 throughout): it reassociates the recurrence
# (decay ratios exp(G_i - G_j) instead of running products, a unit-triangular
# solve per 64-token chunk), so it agrees with the serial oracle to FP32
# rounding accumulated over the tokens: outputs and state <= 2e-5 normwise
# (measured ~1e-6 .. 5e-6).  The conv state is a copy and is exact.
@pytest.mark.parametrize("B,T,K,io", [(1, 64, 4, "f32"), (2, 150, 4, "f32"), (1, 200, 1, "f32"), (1, 300, 2, "f32"),
                                      (2, 130, 4, "bf16"), (3, 1, 4, "f32"), (2, 5, 4, "f32"), (1, 63, 3, "f32")])
def test_gdn_chunked_parity(qw, chunk_ctx, oracle, relerr, B, T, K, io):
    got, ref, st, st_ref, cs, cs_ref = _prefill_case(qw, chunk_ctx, oracle, B, T, K, io, 960 + T)
    bar = 2e-5 if io == "f32" else 4e-3
    print("chunked", B, T, K, io, relerr(got, ref), relerr(st, st_ref))
    assert relerr(got, ref) <= bar, relerr(got, ref)
    assert relerr(st, st_ref) <= 2e-5, relerr(st, st_ref)
    assert np.array_equal(cs, cs_ref)


def test_gdn_chunked_segments(qw, small_ws_ctx, oracle, relerr):
    """T = 300 in 128-token segments (three launches of each kernel)."""
    got, ref, st, st_ref, cs, cs_ref = _prefill_case(qw, small_ws_ctx, oracle, 1, 300, 4, "f32", 970)
    assert relerr(got, ref) <= 2e-5, relerr(got, ref)
    assert relerr(st, st_ref) <= 2e-5, relerr(st, st_ref)
    assert np.array_equal(cs, cs_ref)


def test_gdn_chunked_strong_decay_and_saturated_gates(qw, chunk_ctx, oracle, relerr):
    """Large |A_log| and |a| (decay factors underflow to 0 inside a chunk,
    beta near 0 and 1): the decay ratios stay finite and the result follows
    the serial oracle."""
    B, T, K = 1, 96, 4
    P = _params(oracle, K, 980)
    P["A_log"] = P["A_log"] + 2.5
    dP = {k: dev(v) for k, v in P.items()}
    ld = CD + NH * VD + 2 * NH
    row = oracle.normal((T, ld), 981)
    row[:, CD + NH * VD:] *= 12.0  # a and b far into the saturated ranges
    rows = dev(row)
    cs = np.zeros((B, CD, K - 1), np.float32)
    rs = oracle.normal((B, NH, KD * VD), 982, 0.0, 0.3)
    dcs, drs = dev(cs), dev(rs)
    out = torch.empty(T, NH * VD, device="cuda")
    qw.gdn_prefill(chunk_ctx, dP["conv_w"], dP["A_log"], dP["dt_bias"], dP["norm_w"], rows[:, :CD],
                   rows[:, CD:CD + NH * VD], rows[:, CD + NH * VD:CD + NH * VD + NH], rows[:, CD + NH * VD + NH:],
                   dcs, drs, out, NH, T)
    torch.cuda.synchronize()
    o_ref = np.empty((T, NH * VD), np.float32)
    for t in range(T):
        rt = row[t:t + 1]
        o_ref[t:t + 1], cs, rs = oracle.gdn_step(rt[:, :CD], rt[:, CD + NH * VD:CD + NH * VD + NH],
                                                 rt[:, CD + NH * VD + NH:], rt[:, CD:CD + NH * VD], P["conv_w"],
                                                 P["A_log"], P["dt_bias"], P["norm_w"], cs, rs, NH, KD, VD)
    assert np.isfinite(host(out)).all() and np.isfinite(host(drs)).all()
    assert relerr(host(out), o_ref) <= 2e-5, relerr(host(out), o_ref)
    assert relerr(host(drs), rs) <= 2e-5, relerr(host(drs), rs)


@pytest.mark.parametrize("B,T,K,io", [(1, 7, 4, "f32"), (2, 33, 4, "f32"), (3, 5, 1, "f32"), (2, 9, 4, "bf16")])
def test_gdn_prefill_parity(qw, serial_ctx, oracle, relerr, B, T, K, io):
    """qw_gdn_prefill (serial kernel) over T tokens of B sequences against T
    oracle steps (the serial semantics of the reference forward_batch)."""
    ctx = serial_ctx
    P = _params(oracle, K, 940 + K)
    dP = {k: dev(v) for k, v in P.items()}
    cs = oracle.normal((B, CD, max(K - 1, 0)), 941)
    rs = oracle.normal((B, NH, KD * VD), 942, 0.0, 0.3)
    dcs, drs = dev(cs), dev(rs)
    tdt = torch.float32 if io == "f32" else torch.bfloat16
    ld = CD + NH * VD + 2 * NH
    rows = dev(oracle.normal((B * T, ld), 943), tdt)
    out = torch.empty(B * T, NH * VD, device="cuda", dtype=tdt)
    qw.gdn_prefill(ctx, dP["conv_w"], dP["A_log"], dP["dt_bias"], dP["norm_w"], rows[:, :CD],
                   rows[:, CD:CD + NH * VD], rows[:, CD + NH * VD:CD + NH * VD + NH], rows[:, CD + NH * VD + NH:],
                   dcs, drs, out, NH, T)
    torch.cuda.synchronize()
    r = host(rows).reshape(B, T, ld)
    o_ref = np.empty((B, T, NH * VD), np.float32)
    for t in range(T):
        rt = np.ascontiguousarray(r[:, t])
        o_ref[:, t], cs, rs = oracle.gdn_step(rt[:, :CD], rt[:, CD + NH * VD:CD + NH * VD + NH],
                                              rt[:, CD + NH * VD + NH:], rt[:, CD:CD + NH * VD], P["conv_w"],
                                              P["A_log"], P["dt_bias"], P["norm_w"], cs, rs, NH, KD, VD)
    bar = 1e-5 if io == "f32" else 4e-3
    # the carried state adds a little summation-order difference per token
    sbar = 1e-5 * max(1, T // 8)
    assert relerr(host(out).reshape(B, T, -1), o_ref) <= bar
    assert relerr(host(drs), rs) <= sbar, relerr(host(drs), rs)
    assert np.array_equal(host(dcs), cs)


def test_gdn_prefill_equals_decode_steps(qw, serial_ctx, oracle):
    """One T-token launch of the serial kernel and T one-token launches run
    the same arithmetic: outputs and both states agree bit for bit."""
    ctx = serial_ctx
    B, T, K = 2, 6, 4
    P = {k: dev(v) for k, v in _params(oracle, K, 950).items()}
    cs0 = dev(oracle.normal((B, CD, K - 1), 951))
    rs0 = dev(oracle.normal((B, NH, KD * VD), 952, 0.0, 0.3))
    ld = CD + NH * VD + 2 * NH
    rows = dev(oracle.normal((B, T, ld), 953))

    def parts(x):
        return x[:, :CD], x[:, CD:CD + NH * VD], x[:, CD + NH * VD:CD + NH * VD + NH], x[:, CD + NH * VD + NH:]

    cs1, rs1 = cs0.clone(), rs0.clone()
    out1 = torch.empty(B * T, NH * VD, device="cuda")
    qw.gdn_prefill(ctx, P["conv_w"], P["A_log"], P["dt_bias"], P["norm_w"], *parts(rows.reshape(B * T, ld)), cs1,
                   rs1, out1, NH, T)
    cs2, rs2 = cs0.clone(), rs0.clone()
    out2 = torch.empty(B, T, NH * VD, device="cuda")
    for t in range(T):
        o = torch.empty(B, NH * VD, device="cuda")
        qw.gdn_decode(ctx, P["conv_w"], P["A_log"], P["dt_bias"], P["norm_w"], *parts(rows[:, t]), cs2, rs2, o, NH)
        out2[:, t] = o
    torch.cuda.synchronize()
    assert torch.equal(out1, out2.reshape(B * T, -1))
    assert torch.equal(rs1, rs2) and torch.equal(cs1, cs2)


def test_gdn_prefill_errors(qw, ctx):
    P = {"conv_w": torch.zeros(CD, 4, device="cuda"), "A_log": torch.zeros(NH, device="cuda"),
         "dt_bias": torch.zeros(NH, device="cuda"), "norm_w": torch.ones(VD, device="cuda")}
    x = torch.zeros(6, CD, device="cuda")
    out = torch.empty(6, NH * VD, device="cuda")
    cs = torch.zeros(1, CD * 3, device="cuda")
    rs = torch.zeros(1, NH * KD * VD, device="cuda")
    with pytest.raises(qw.QwError):  # 6 rows are not whole 4-token sequences
        qw.gdn_prefill(ctx, P["conv_w"], P["A_log"], P["dt_bias"], P["norm_w"], x, x, x, x, cs, rs, out, NH, 4)
    with pytest.raises(qw.QwError):  # zero tokens
        qw.gdn_prefill(ctx, P["conv_w"], P["A_log"], P["dt_bias"], P["norm_w"], x, x, x, x, cs, rs, out, NH, 0)
