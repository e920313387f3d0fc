"""The whole greedy decode step (qwen3.5_0.8b_deploy_amd/engine.py) on the GPU
against the CPU oracle composed of its pinned pieces (orc_rmsnorm,
orc_linear_f32, orc_gdn_step, orc_full_attn_seq, orc_mlp, orc_lmhead_argmax),
layer by layer in the reference LanguageBackbone order
(language_backbone.cpp:54-88).

Model: the real layer shapes (hidden 1024, MLP 3584, 16-head Gated-DeltaNet,
8/2-head full attention) with 4 layers in the reference pattern (linear,
linear, linear, full) and a 2048-token vocabulary so that the CPU oracle runs
in seconds; FP32 weights, FP32 KV cache, FP32 embedding.  3 sequences, 6
greedy tokens each, token ids fed back on the device (the captured step is
replayed, so the graph path is what is tested).

Bars: token ids identical whenever the oracle's top-2 logit gap exceeds 1e-3
(random weights: gaps are far larger); the hidden state after the last step
within 1e-4 normwise (FP32 everywhere, only reduction orders differ).
"""
import importlib.util
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def host(t):
    return t.float().cpu().numpy()

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _engine_mod():
    spec = importlib.util.spec_from_file_location("qw_engine", os.path.join(ROOT, "qwen3.5_0.8b_deploy_amd", "engine.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def make_layers(oracle, n_layers, seed, std=0.03):
    from math import prod
    em = _engine_mod()
    layers = []
    for i in range(n_layers):
        s = seed + 100 * i
        L = {"in_norm": oracle.normal((em.H,), s, 0.0, 0.1), "post_norm": oracle.normal((em.H,), s + 1, 0.0, 0.1),
             "gate": oracle.normal((em.I, em.H), s + 2, 0.0, std), "up": oracle.normal((em.I, em.H), s + 3, 0.0, std),
             "down": oracle.normal((em.H, em.I), s + 4, 0.0, std)}
        if em.is_linear_layer(i):
            L.update(qkv=oracle.normal((em.CD, em.H), s + 5, 0.0, std), a=oracle.normal((em.LNH, em.H), s + 6, 0.0, std),
                     b=oracle.normal((em.LNH, em.H), s + 7, 0.0, std),
                     z=oracle.normal((em.LNH * em.VD, em.H), s + 8, 0.0, std),
                     conv=oracle.normal((em.CD, em.CK), s + 9, 0.0, 0.5),
                     out=oracle.normal((em.H, em.LNH * em.VD), s + 10, 0.0, std),
                     A_log=oracle.normal((em.LNH,), s + 11, 0.0, 0.5), dt_bias=oracle.normal((em.LNH,), s + 12, 0.0, 0.5),
                     norm_w=1.0 + oracle.normal((em.VD,), s + 13, 0.0, 0.1))
        else:
            L.update(q=oracle.normal((em.FNH * 2 * em.HD, em.H), s + 5, 0.0, std),
                     k=oracle.normal((em.FNKV * em.HD, em.H), s + 6, 0.0, std),
                     v=oracle.normal((em.FNKV * em.HD, em.H), s + 7, 0.0, std),
                     q_norm=oracle.normal((em.HD,), s + 8, 0.0, 0.1), k_norm=oracle.normal((em.HD,), s + 9, 0.0, 0.1),
                     o=oracle.normal((em.H, em.FNH * em.HD), s + 10, 0.0, std))
        layers.append(L)
    return layers


class OracleModel:
    """The same decode, token by token, on the CPU oracle (one sequence)."""

    def __init__(self, oracle, layers, final_norm, embed, capacity):
        self.o, self.layers, self.final_norm, self.embed = oracle, layers, final_norm, embed
        em = _engine_mod()
        self.em = em
        self.state = []
        for i, L in enumerate(layers):
            if em.is_linear_layer(i):
                self.state.append([np.zeros((1, em.CD, em.CK - 1), np.float32),
                                   np.zeros((1, em.LNH, em.KD * em.VD), np.float32)])
            else:
                self.state.append([(np.zeros((capacity, em.FNKV, em.HD), np.float32),
                                    np.zeros((capacity, em.FNKV, em.HD), np.float32),
                                    np.zeros((capacity, em.FNKV), np.float32), np.zeros((capacity, em.FNKV), np.float32))])

    def step(self, token, pos):
        o, em = self.o, self.em
        x = self.embed[token][None].astype(np.float32)
        for i, L in enumerate(self.layers):
            xn = o.rmsnorm(x, L["in_norm"])
            if em.is_linear_layer(i):
                mixed, z = o.linear(L["qkv"], xn), o.linear(L["z"], xn)
                a, b = o.linear(L["a"], xn), o.linear(L["b"], xn)
                cs, rs = self.state[i]
                core, cs, rs = o.gdn_step(mixed, a, b, z, L["conv"], L["A_log"], L["dt_bias"], L["norm_w"], cs, rs,
                                          em.LNH, em.KD, em.VD)
                self.state[i] = [cs, rs]
                x = x + o.linear(L["out"], core)
            else:
                qr = o.linear(L["q"], xn).reshape(1, em.FNH, 2, em.HD)
                q = np.ascontiguousarray(qr[:, :, 0].reshape(1, -1))
                g = np.ascontiguousarray(qr[:, :, 1].reshape(1, -1))
                k, v = o.linear(L["k"], xn), o.linear(L["v"], xn)
                core, cache = o.full_attn_seq(q, g, k, v, L["q_norm"], L["k_norm"], em.FNH, em.FNKV, em.HD,
                                              pos0=pos, cache=self.state[i][0])
                x = x + o.linear(L["o"], core)
            x = x + o.mlp(L["gate"], L["up"], L["down"], o.rmsnorm(x, L["post_norm"]))
        h = o.rmsnorm(x, self.final_norm)
        logits = o.linear(self.embed, h)[0]
        top = np.sort(logits)[-2:]
        ids, _ = o.lmhead_argmax(self.embed, h)
        return int(ids[0]), float(top[1] - top[0]), x[0]


def test_engine_greedy_matches_oracle(qw, ctx, oracle, relerr):
    em = _engine_mod()
    B, steps, V, cap = 3, 6, 2048, 16
    layers = make_layers(oracle, 4, 3000)
    final_norm = oracle.normal((em.H,), 2999, 0.0, 0.1)
    embed = oracle.normal((V, em.H), 2998, 0.0, 1.0)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    eng = em.DecodeEngine(qw, ctx, [{k: dev(v) for k, v in L.items()} for L in layers], dev(final_norm), dev(embed), B,
                          cap, fmt=qw.WFMT_F32, lm_fmt=qw.WFMT_F32, kv_int8=False)
    starts = [5, 77, 1999]
    eng.reset(starts)
    stream = torch.cuda.Stream()
    g = qw.Graph(ctx, stream)
    with torch.cuda.stream(stream):
        with g:
            eng.step(stream=stream)
    gpu_ids = []
    for _ in range(steps):
        g.launch(stream)
        stream.synchronize()
        gpu_ids.append(eng.ids.cpu().numpy().copy())
    assert ctx.device_error() == 0
    assert eng.pos.cpu().tolist() == [steps] * B
    x_gpu = eng.x.cpu().numpy()
    for b in range(B):
        om = OracleModel(oracle, layers, final_norm, embed, cap)
        tok = starts[b]
        for t in range(steps):
            nxt, gap, x = om.step(tok, t)
            if gap > 1e-3:
                assert gpu_ids[t][b] == nxt, (b, t, gpu_ids[t][b], nxt, gap)
            tok = int(gpu_ids[t][b])  # follow the GPU's choice
        assert relerr(x_gpu[b], x) <= 1e-4, relerr(x_gpu[b], x)


def test_engine_eager_equals_graph(qw, ctx, oracle):
    """The captured step replays the eager step exactly (same ids, same state)."""
    em = _engine_mod()
    B, V = 2, 1024
    layers = make_layers(oracle, 4, 4000)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    tl = [{k: dev(v) for k, v in L.items()} for L in layers]
    fn, emb = dev(oracle.normal((em.H,), 4999, 0.0, 0.1)), dev(oracle.normal((V, em.H), 4998)).bfloat16()
    e1 = em.DecodeEngine(qw, ctx, tl, fn, emb, B, 8)
    e2 = em.DecodeEngine(qw, ctx, tl, fn, emb, B, 8)
    e1.reset([3, 4])
    e2.reset([3, 4])
    stream = torch.cuda.Stream()
    g = qw.Graph(ctx, stream)
    with torch.cuda.stream(stream):
        with g:
            e2.step(stream=stream)
        for _ in range(4):
            e1.step(stream=stream)
            g.launch(stream)
            stream.synchronize()
            assert torch.equal(e1.ids, e2.ids) and torch.equal(e1.x, e2.x)


def test_engine_norm_first_matches_prologue(qw, ctx, oracle, relerr):
    """BF16 engine: RMSNorm once into a BF16 buffer (the path for more than 12
    sequences) against the projections' own RMSNorm prologue on the FP32
    residual stream (the few-sequence path), same weights and tokens.  The
    only difference is x rounded to BF16 before the projections (the
    prologue keeps it as a BF16 hi + lo pair), so the hidden states agree to
    the BF16 bar (1e-2) and the greedy ids agree wherever the two engines
    saw the same history."""
    em = _engine_mod()
    B, V = 6, 1024
    layers = make_layers(oracle, 4, 5000)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    tl = [{k: dev(v) for k, v in L.items()} for L in layers]
    fn, emb = dev(oracle.normal((em.H,), 5999, 0.0, 0.1)), dev(oracle.normal((V, em.H), 5998)).bfloat16()
    e1 = em.DecodeEngine(qw, ctx, tl, fn, emb, B, 8, norm_first=True)
    e2 = em.DecodeEngine(qw, ctx, tl, fn, emb, B, 8, norm_first=False)
    assert e1.norm_first and not e2.norm_first
    start = [3, 4, 100, 511, 7, 1000]
    e1.reset(start)
    e2.reset(start)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        e1.step(stream=stream)
        e2.step(stream=stream)
        stream.synchronize()
    assert ctx.device_error() == 0
    x1, x2 = e1.x.cpu().numpy(), e2.x.cpu().numpy()
    for b in range(B):
        assert relerr(x1[b], x2[b].astype(np.float64)) <= 1e-2, (b, relerr(x1[b], x2[b].astype(np.float64)))
    # the automatic choice: norm-first only for BF16 weights above 12 sequences
    assert em.DecodeEngine(qw, ctx, tl, fn, emb, 13, 8).norm_first
    assert not em.DecodeEngine(qw, ctx, tl, fn, emb, 12, 8).norm_first


def test_engine_prefill_matches_steps(qw, ctx, oracle, relerr):
    """prefill(T tokens) == T teacher-forced decode steps: the same next ids,
    last hidden state, Gated-DeltaNet states and KV caches, then the same
    greedy continuation.  FP32 weights and cache; T = 40 takes the chunked
    Gated-DeltaNet (>= 24 tokens) and the query-block attention (>= 16), each
    pinned separately against the serial kernels at 2e-5; bar 1e-4."""
    em = _engine_mod()
    B, T, V, cap = 2, 40, 1024, 64
    layers = make_layers(oracle, 4, 6000)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    tl = [{k: dev(v) for k, v in L.items()} for L in layers]
    fn, emb = dev(oracle.normal((em.H,), 6999, 0.0, 0.1)), dev(oracle.normal((V, em.H), 6998))
    kw = dict(fmt=qw.WFMT_F32, lm_fmt=qw.WFMT_F32, kv_int8=False)
    ea = em.DecodeEngine(qw, ctx, tl, fn, emb, B, cap, **kw)
    eb = em.DecodeEngine(qw, ctx, tl, fn, emb, B, cap, **kw)
    prompt = torch.from_numpy(np.random.default_rng(7).integers(0, V, (B, T)).astype(np.int32)).cuda()
    ea.reset([0] * B)
    eb.reset([0] * B)
    ea.prefill(prompt)
    for t in range(T):
        eb.ids.copy_(prompt[:, t])
        eb.step()
    torch.cuda.synchronize()
    assert ctx.device_error() == 0
    assert ea.pos.tolist() == [T] * B and eb.pos.tolist() == [T] * B
    assert torch.equal(ea.ids, eb.ids), (ea.ids, eb.ids)
    assert relerr(host(ea.x), host(eb.x).astype(np.float64)) <= 1e-4
    for Pa, Pb in zip(ea.layers, eb.layers):
        if Pa["linear"]:
            assert relerr(host(Pa["rs"]), host(Pb["rs"]).astype(np.float64)) <= 1e-4
            assert relerr(host(Pa["cs"]), host(Pb["cs"]).astype(np.float64)) <= 1e-4
        else:
            for ca, cb in zip(Pa["cache"][:2], Pb["cache"][:2]):
                assert relerr(host(ca[:, :T]), host(cb[:, :T]).astype(np.float64)) <= 1e-4
    for _ in range(3):  # the greedy continuation agrees
        ea.step()
        eb.step()
        torch.cuda.synchronize()
        assert torch.equal(ea.ids, eb.ids)


@pytest.mark.parametrize("norm_first", [False, True])
def test_engine_bf16_matches_oracle(qw, ctx, oracle, relerr, norm_first):
    """The production weight format: BF16 weights (the norms and the
    Gated-DeltaNet parameters stay FP32) against the oracle run on the same
    BF16-rounded matrices (FP32 cache on both sides).  The engine also rounds
    the attention / Gated-DeltaNet output and the MLP intermediate to BF16
    (the MFMA input type of the next projection), and with norm_first the
    normalized layer inputs, so the bar is the BF16 one: 1e-2 on the hidden
    state; greedy ids equal wherever the oracle's top-2 gap exceeds 0.05."""
    em = _engine_mod()
    B, steps, V, cap = 3, 4, 2048, 16
    layers = make_layers(oracle, 4, 8000)
    final_norm = oracle.normal((em.H,), 8999, 0.0, 0.1)
    embed = oracle.normal((V, em.H), 8998, 0.0, 1.0)
    matrices = ("gate", "up", "down", "qkv", "a", "b", "z", "out", "q", "k", "v", "o")
    rounded = [{k: (oracle.round_bf16(v) if k in matrices else v) for k, v in L.items()} for L in layers]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    eng = em.DecodeEngine(qw, ctx, [{k: dev(v) for k, v in L.items()} for L in layers], dev(final_norm), dev(embed), B,
                          cap, fmt=qw.WFMT_BF16, lm_fmt=qw.WFMT_BF16, kv_int8=False, norm_first=norm_first)
    starts = [11, 500, 2047]
    eng.reset(starts)
    gpu_ids = []
    for _ in range(steps):
        eng.step()
        torch.cuda.synchronize()
        gpu_ids.append(eng.ids.cpu().numpy().copy())
    assert ctx.device_error() == 0
    x_gpu = eng.x.cpu().numpy()
    emb_r = oracle.round_bf16(embed)
    for b in range(B):
        om = OracleModel(oracle, rounded, final_norm, embed, cap)
        om.embed = embed  # the gather reads the FP32 table; the lm_head below the BF16 copy
        tok = starts[b]
        for t in range(steps):
            nxt, gap, x = om.step(tok, t)
            h = oracle.rmsnorm(x[None], final_norm)
            logits = oracle.linear(emb_r, h)[0]
            top = np.sort(logits)[-2:]
            if top[1] - top[0] > 0.05:
                assert gpu_ids[t][b] == int(np.argmax(logits)), (b, t, gpu_ids[t][b], int(np.argmax(logits)))
            tok = int(gpu_ids[t][b])
        err = relerr(x_gpu[b], x)
        print("bf16 engine", norm_first, b, err)
        assert err <= 1e-2, err


def test_engine_check_raises_on_device_error(qw, ctx, oracle, relerr):
    """A token past the KV cache raises the device flag; the eager step reads
    it and raises.  The read clears the flag (and returns the one-launch MLP's
    counters to zero), after which a one-launch MLP is exact again."""
    em = _engine_mod()
    B, V, cap = 1, 512, 2
    layers = make_layers(oracle, 4, 9000)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    tl = [{k: dev(v) for k, v in L.items()} for L in layers]
    fn, emb = dev(oracle.normal((em.H,), 9999, 0.0, 0.1)), dev(oracle.normal((V, em.H), 9998)).bfloat16()
    eng = em.DecodeEngine(qw, ctx, tl, fn, emb, B, cap)
    eng.reset([3], positions=[cap - 1])
    eng.step()                      # position cap-1: inside the cache
    with pytest.raises(RuntimeError, match="device error flag"):
        eng.step()                  # position cap: outside
    assert ctx.device_error() == 0
    # the one-launch MLP after the reset of its counters
    H, I = em.H, em.I
    G, U, D = (oracle.normal(s, 9100 + i, 0.0, 0.02) for i, s in enumerate([(I, H), (I, H), (H, I)]))
    gu = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16)
    dn = qw.Weight.pack(ctx, D, qw.WFMT_BF16)
    x = dev(oracle.normal((1, H), 9103)).bfloat16()
    for _ in range(2):
        y = torch.empty(1, H, device="cuda")
        qw.mlp_fused(ctx, gu, dn, x, y, gamma=None, residual=x)
        torch.cuda.synchronize()
        ref = oracle.mlp_f64(oracle.round_bf16(G), oracle.round_bf16(U), oracle.round_bf16(D), host(x)) + host(x)
        assert relerr(host(y), ref) <= 2e-3
    assert ctx.device_error() == 0
