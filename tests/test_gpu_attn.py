"""GPU parity of the gated full-attention core (qw_attn_forward) against the
CPU oracle (orc_full_attn_seq, pinned bit-exactly to the reference's own
FullAttention::forward in tests/test_oracle.py).

Shapes: Qwen3.5-0.8B full attention, 8 query heads, 2 KV heads, head dim 256,
rotary 64 dims, theta 1e7 (also head dim 128 and theta 100 for large angles).
Sequences are prefilled and then decoded through the GPU cache; the oracle
runs the same token stream through its own cache.

Bars (normwise relative error against the oracle):
  FP32 cache, FP32 io      2e-5: only reduction orders (norms, dot products,
                           online softmax), __expf and the device cosf/sinf
                           differ; measured ~1e-6.
  INT8 cache               5e-3: the same, plus f16 MFMA operands for q and
                           p (2^-11; measured ~2.5e-4), plus INT8
                           rounding flips where the
                           GPU's and the oracle's normalized k or v land on
                           either side of a .5 step (one step = 1/127 of the
                           head's max); the cached codes are checked to differ
                           by at most one step, on at most 1% of entries.
  BF16 io                  1e-2: inputs rounded identically for both sides; the
                           output carries one BF16 rounding.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

NH, NKV, HD, ROT = 8, 2, 256, 64


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


class Stream:
    """B sequences of raw projections, one stacked row per token:
    [q0 g0 q1 g1 ... q7 g7 | k | v] (the interleaved Q|gate projection output)."""

    def __init__(self, oracle, B, T, seed, hd=HD, nh=NH, nkv=NKV):
        self.hd, self.nh, self.nkv = hd, nh, nkv
        self.ld = nh * 2 * hd + 2 * nkv * hd
        self.rows = oracle.normal((B, T, self.ld), seed)
        self.qn = oracle.normal((hd,), seed + 1, 0.0, 0.1)
        self.kn = oracle.normal((hd,), seed + 2, 0.0, 0.1)

    def parts(self, rows):
        """(q, gate, k, v) numpy arrays of rows [..., ld] for the oracle."""
        nh, hd, nkv = self.nh, self.hd, self.nkv
        qg = rows[..., :nh * 2 * hd].reshape(rows.shape[:-1] + (nh, 2, hd))
        q = qg[..., 0, :].reshape(rows.shape[:-1] + (nh * hd,))
        g = qg[..., 1, :].reshape(rows.shape[:-1] + (nh * hd,))
        k = rows[..., nh * 2 * hd:nh * 2 * hd + nkv * hd]
        v = rows[..., nh * 2 * hd + nkv * hd:]
        return [np.ascontiguousarray(x) for x in (q, g, k, v)]

    def views(self, drows):
        """(q, gate, k, v) device views of rows [R, ld]: q at head stride 2*hd."""
        nh, hd, nkv = self.nh, self.hd, self.nkv
        return drows[:, 0:], drows[:, hd:], drows[:, nh * 2 * hd:], drows[:, nh * 2 * hd + nkv * hd:]


def run_gpu(qw, ctx, st, cache, drows, pos, tokens, theta, rot, out_dtype=torch.float32, max_len=0):
    q, g, k, v = st.views(drows)
    out = torch.empty(drows.shape[0], st.nh * st.hd, device="cuda", dtype=out_dtype)
    qw.attn_forward(ctx, dev(st.qn), dev(st.kn), cache, dev(np.array(pos, np.int32), torch.int32), q, g, k, v, out,
                    num_heads=st.nh, num_kv_heads=st.nkv, head_dim=st.hd, rotary_dim=rot, rope_theta=theta,
                    tokens=tokens, q_head_stride=2 * st.hd, max_len=max_len)
    return out


def oracle_stream(oracle, st, rows_b, int8, theta, rot, capacity):
    """All tokens of one sequence through the oracle (its own cache)."""
    q, g, k, v = st.parts(rows_b)
    out, cache = oracle.full_attn_seq(q, g, k, v, st.qn, st.kn, st.nh, st.nkv, st.hd, rotary_dim=rot, theta=theta,
                                      int8=int8, capacity=capacity)
    return out, cache


@pytest.mark.parametrize("int8,io,hd,theta", [(False, "f32", 256, 1.0e7), (True, "f32", 256, 1.0e7),
                                              (True, "bf16", 256, 1.0e7), (False, "f32", 128, 100.0),
                                              (True, "f32", 128, 100.0)])
def test_attn_prefill_then_decode(qw, ctx, oracle, relerr, int8, io, hd, theta):
    """3 sequences: a 37-token prefill (one launch over all 111 rows, causal
    within each sequence), then 5 decode steps of one token each."""
    B, T0, steps, cap = 3, 37, 5, 64
    rot = hd // 4
    st = Stream(oracle, B, T0 + steps, 200 + hd + int(int8), hd=hd)
    tdt = torch.float32 if io == "f32" else torch.bfloat16
    rows = st.rows if io == "f32" else host(dev(st.rows, torch.bfloat16))  # what the GPU sees
    cache = qw.kv_cache(B, cap, st.nkv, hd, int8=int8)
    outs = [run_gpu(qw, ctx, st, cache, dev(st.rows[:, :T0].reshape(B * T0, -1), tdt), [0] * B, T0, theta, rot,
                    out_dtype=tdt)]
    for s in range(steps):
        outs.append(run_gpu(qw, ctx, st, cache, dev(st.rows[:, T0 + s], tdt), [T0 + s] * B, 1, theta, rot,
                            out_dtype=tdt))
    torch.cuda.synchronize()
    got = np.concatenate([host(outs[0]).reshape(B, T0, -1)] + [host(o)[:, None] for o in outs[1:]], axis=1)
    bar = (5e-3 if int8 else 2e-5) if io == "f32" else 1e-2
    for b in range(B):
        ref, (kc, vc, ks, vs) = oracle_stream(oracle, st, rows[b], int8, theta, rot, cap)
        err = relerr(got[b], ref)
        print("attn", int8, io, hd, b, err)
        assert err <= bar, (b, err)
        gk, gv = host(cache[0][b]), host(cache[1][b])
        n = T0 + steps
        if int8:
            for gc, oc in ((gk, kc), (gv, vc)):
                d = np.abs(gc[:n].astype(np.int32) - oc[:n].astype(np.int32))
                assert d.max() <= 1 and (d > 0).mean() <= 0.01, (d.max(), (d > 0).mean())
            np.testing.assert_allclose(host(cache[2][b])[:n], ks[:n], rtol=2e-5)
            np.testing.assert_allclose(host(cache[3][b])[:n], vs[:n], rtol=2e-5)
        else:
            assert relerr(gk[:n], kc[:n]) <= 2e-5 and relerr(gv[:n], vc[:n]) <= 2e-5


def test_attn_ragged_positions(qw, ctx, oracle, relerr):
    """Sequences at different positions in one decode launch: each attends to
    exactly its own prefix (positions 0, 9 and 30)."""
    B, cap = 3, 48
    lens = [1, 10, 31]
    st = Stream(oracle, B, max(lens), 300)
    cache = qw.kv_cache(B, cap, int8=False)
    # prefill each sequence to lens[b]-1 tokens with its own launch, then one decode step for all
    for b in range(B):
        n = lens[b] - 1
        if n:
            sub = tuple(c[b:b + 1] for c in cache)
            run_gpu(qw, ctx, st, sub, dev(st.rows[b, :n]), [0], n, 1.0e7, ROT)
    out = run_gpu(qw, ctx, st, cache, dev(np.stack([st.rows[b, lens[b] - 1] for b in range(B)])),
                  [n - 1 for n in lens], 1, 1.0e7, ROT)
    torch.cuda.synchronize()
    for b in range(B):
        ref, _ = oracle_stream(oracle, st, st.rows[b, :lens[b]], False, 1.0e7, ROT, cap)
        assert relerr(host(out)[b], ref[-1]) <= 2e-5


@pytest.mark.parametrize("int8", [False, True])
def test_attn_long_context_decode(qw, ctx, oracle, relerr, int8):
    """A 3000-token cache built by one GPU prefill, then a decode step split
    over many key ranges: checked against the oracle's attention over the
    GPU-written cache (dequantized with its own scales) and the oracle's
    norm + RoPE of the new token."""
    L, cap = 3000, 3072
    st = Stream(oracle, 1, L + 1, 400)
    cache = qw.kv_cache(1, cap, int8=int8)
    run_gpu(qw, ctx, st, cache, dev(st.rows[0, :L]), [0], L, 1.0e7, ROT)
    out = run_gpu(qw, ctx, st, cache, dev(st.rows[0, L:L + 1]), [L], 1, 1.0e7, ROT)
    torch.cuda.synchronize()
    q, g, k, v = st.parts(st.rows[0, L:L + 1])
    qn, _ = oracle.attn_norm_rope(q[0], k[0], st.qn, st.kn, L, NH, NKV, HD, ROT, 1.0e7)
    kc, vc = host(cache[0][0, :L + 1]), host(cache[1][0, :L + 1])
    if int8:
        kc = kc * host(cache[2][0, :L + 1])[..., None]
        vc = vc * host(cache[3][0, :L + 1])[..., None]
    ref = oracle.attn_token(qn, g[0], kc, vc, NH, NKV, HD)
    # INT8 cache: f16 MFMA operands for q and p (2^-11); FP32 cache: FP32 throughout
    assert relerr(host(out)[0], ref) <= (5e-3 if int8 else 2e-5)


def test_attn_position_outside_cache_flags(qw, ctx, oracle):
    """A token past the capacity writes nothing, outputs zeros and sets the
    device error flag; the other sequence in the launch is unaffected."""
    st = Stream(oracle, 2, 1, 500)
    cache = qw.kv_cache(2, 8, int8=True)
    ctx.device_error()  # clear
    out = run_gpu(qw, ctx, st, cache, dev(st.rows[:, 0]), [0, 8], 1, 1.0e7, ROT)
    torch.cuda.synchronize()
    assert ctx.device_error() != 0
    assert not host(out)[1].any() and host(out)[0].any()
    assert not host(cache[0][1]).any()



def test_attn_repeatable(qw, ctx, oracle):
    st = Stream(oracle, 2, 20, 600)
    outs = []
    for _ in range(3):
        cache = qw.kv_cache(2, 32, int8=True)
        outs.append(run_gpu(qw, ctx, st, cache, dev(st.rows.reshape(40, -1)), [0, 0], 20, 1.0e7, ROT))
    torch.cuda.synchronize()
    assert all(torch.equal(outs[0], o) for o in outs[1:])


def test_attn_errors(qw, ctx, oracle):
    st = Stream(oracle, 1, 1, 700)
    cache = qw.kv_cache(1, 8, int8=False)
    with pytest.raises(qw.QwError):  # 5 query heads per KV head
        run_gpu(qw, ctx, Stream(oracle, 1, 1, 701, nh=10), cache, dev(Stream(oracle, 1, 1, 701, nh=10).rows[:, 0]),
                [0], 1, 1.0e7, ROT)
    with pytest.raises(qw.QwError):  # odd rotary dim
        run_gpu(qw, ctx, st, cache, dev(st.rows[:, 0]), [0], 1, 1.0e7, 63)


def _ctx_with(qw, env, **kw):
    import os
    os.environ.update(env)
    try:
        return qw.Context(0, **kw)
    finally:
        for k in env:
            del os.environ[k]


@pytest.mark.parametrize("int8", [True, False])
def test_attn_prefill_kernel_matches_split_path(qw, oracle, relerr, int8):
    """The query-block prefill kernel, the key-split kernel (a context that
    sends every run to it) and, with a 6 MB workspace, the prefill kernel in
    768-token chunks of one sequence give the same result: 2 sequences of
    1000 tokens, the second starting at position 7 after a 7-token prefix.
    Over an INT8 cache the prefill kernel runs f16 MFMAs (q and p rounded to
    f16, 2^-11), so it meets the split path within the INT8 bar (5e-3); over
    an FP32 cache both are FP32 (2e-5); the chunked run is the same kernel."""
    B, T, cap = 2, 1000, 1024
    st = Stream(oracle, B, T + 7, 800)
    outs = []
    ctxs = [_ctx_with(qw, {}), _ctx_with(qw, {"QW_ATTN_PREFILL_MIN": "100000"}),
            _ctx_with(qw, {}, workspace_bytes=qw.lib().qw_workspace_query(1, 1, 1) + (6 << 20))]
    for c in ctxs:
        cache = qw.kv_cache(B, cap, int8=int8)
        sub = tuple(x[1:2] for x in cache)
        run_gpu(qw, c, st, sub, dev(st.rows[1, :7]), [0], 7, 1.0e7, ROT)
        rows = np.stack([st.rows[0, :T], st.rows[1, 7:T + 7]]).reshape(B * T, -1)
        outs.append(host(run_gpu(qw, c, st, cache, dev(rows), [0, 7], T, 1.0e7, ROT)))
        torch.cuda.synchronize()
    for c in ctxs:
        c.close()
    print("prefill vs split", int8, relerr(outs[1], outs[0]), relerr(outs[2], outs[0]))
    assert relerr(outs[1], outs[0]) <= (5e-3 if int8 else 2e-5) and relerr(outs[2], outs[0]) <= 2e-5
    ref0, _ = oracle_stream(oracle, st, st.rows[0, :200], int8, 1.0e7, ROT, cap)
    assert relerr(outs[0][:200], ref0) <= (5e-3 if int8 else 2e-5)


@pytest.mark.parametrize("io", ["f32", "bf16"])
def test_attn_one_launch_decode_matches_three_launches(qw, oracle, io):
    """One new token per sequence over an INT8 cache runs as one launch (the
    attention kernel normalizes q, writes the new K/V and merges its splits
    itself).  It computes exactly what the prep / split / combine launches
    compute: the same outputs and the same cache contents, bit for bit, over
    a prefill and 6 decode steps of 3 sequences at ragged positions -- short
    rows (one split) and long rows (9 splits) in the same launches."""
    B, cap = 3, 1200
    starts = [5, 300, 1100]
    st = Stream(oracle, B, max(starts) + 6, 900)
    tdt = torch.float32 if io == "f32" else torch.bfloat16
    res = []
    for env in ({}, {"QW_ATTN_FUSED": "0"}):
        c = _ctx_with(qw, env)
        cache = qw.kv_cache(B, cap, int8=True)
        for b in range(B):  # prefill each sequence's prefix (same kernels for both contexts)
            sub = tuple(x[b:b + 1] for x in cache)
            run_gpu(qw, c, st, sub, dev(st.rows[b, :starts[b]], tdt), [0], starts[b], 1.0e7, ROT)
        outs = []
        for s in range(6):
            rows = np.stack([st.rows[b, starts[b] + s] for b in range(B)])
            outs.append(run_gpu(qw, c, st, cache, dev(rows, tdt), [p + s for p in starts], 1, 1.0e7, ROT,
                                out_dtype=tdt))
        torch.cuda.synchronize()
        assert c.device_error() == 0
        res.append(([o.clone() for o in outs], [x.clone() for x in cache]))
        c.close()
    (o1, c1), (o0, c0) = res
    for s in range(6):
        assert torch.equal(o1[s], o0[s]), s
    for x1, x0 in zip(c1, c0):
        assert torch.equal(x1, x0)
