"""CPU tests of the oracle (oracle/qw_oracle.c): it is pinned here before any
GPU result is compared with it.

Pins, by function:
  number formats      numpy float16 (IEEE RNE), torch bfloat16 (RNE), hand-made
                      bit patterns (ties, overflow, subnormals, NaN)
  MT19937-64          the C++ standard's known answer (10000th output of the
                      default seed) and the published first output
  linear (FP32)       the reference's LMHead::forward compiled from its source
                      (golden vectors + oracle/_ref), numpy float64, closed forms
  quantize recipe     hand-worked golden rows (tests/golden/quant.npz)
  INT8 dequant GEMV   exact integer arithmetic with power-of-two scales
  RMSNorm (1+w)       constant-vector closed form, the reference unit test's
                      uniform-input known answer, numpy float64
  residual + RMSNorm  exact sum, then the RMSNorm pin
  MLP                 reference MLP::forward_batch (golden + oracle/_ref),
                      numpy float64 composition
  Q/gate split        index identity on an arange input
  argmax / lm_head    the reference Sampler (golden ties), planted maxima,
                      numpy float64 argmax with a clear top-2 gap
  Gated-DeltaNet      reference LinearAttention::forward (golden + oracle/_ref),
                      numpy float64 matrix form, closed forms (beta -> 0, unit tap)
  full attention      reference FullAttention::forward (golden + oracle/_ref),
                      numpy float64 statement, closed forms (position 0, a
                      single cached token, constant input, rotation norms)
  INT8 KV recipe      vectors worked by hand (ties away from zero, +-127, tiny
                      and zero heads)
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def np_silu(v):
    return v / (1.0 + np.exp(-v))


# ---- number formats --------------------------------------------------------
def test_f16_matches_numpy(oracle):
    x = np.concatenate([
        oracle.normal(4096, 1, 0.0, 3.0),
        np.array([0.0, -0.0, 1.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32),
    ]).astype(np.float32)
    got = oracle.to_f16(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    assert np.array_equal(oracle.from_f16(ref), ref.view(np.float16).astype(np.float32))


def test_bf16_bits(oracle):
    torch = pytest.importorskip("torch")
    x = np.concatenate([
        oracle.normal(4096, 2, 0.0, 10.0),
        np.array([1.0, -1.0, 3.3895314e38, -3.4e38], np.float32),
    ]).astype(np.float32)
    # exact ties: lower 16 bits 0x8000, with even and odd kept mantissa
    ties = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x40490000 | 0x8000], np.uint32).view(np.float32)
    x = np.concatenate([x, ties])
    got = oracle.to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    assert list(oracle.to_bf16(ties)) == [0x3F80, 0x3F82, 0xBF80, 0x404A]
    back = oracle.from_bf16(got)
    assert np.array_equal(back.view(np.uint32) >> 16, got.astype(np.uint32))
    assert np.isnan(oracle.round_bf16(np.array([np.nan], np.float32))[0])


# ---- generator ---------------------------------------------------------------
def test_mt19937_64_known_answers(oracle):
    r = oracle.mt64_raw(5489, 10000)
    assert int(r[0]) == 14514284786278117030
    assert int(r[-1]) == 9981545732273789042  # C++ [rand.predef]


def test_normal_fill_moments(oracle):
    v = oracle.normal(200000, 0, 0.0, 1.0).astype(np.float64)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    u = oracle.uniform(100000, 3, 1e-3, 2e-2)
    assert u.min() >= 1e-3 and u.max() <= 2e-2
    q = oracle.int8_uniform(100000, 4)
    assert q.min() == -127 and q.max() == 127


# ---- projections -----------------------------------------------------------
def test_linear_matches_reference_golden(oracle):
    g = np.load(os.path.join(GOLDEN, "ref_ops.npz"))
    y = oracle.linear(g["lin_W"], g["lin_x"])
    assert np.array_equal(y, g["lin_y"])  # same ascending-k FP32 loop


def test_linear_fp64_and_closed_forms(oracle):
    N, K = 40, 192
    W = oracle.normal((N, K), 5, 0.0, 0.02)
    x = oracle.normal((4, K), 6)
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    assert np.abs(oracle.linear_f64(W, x) - ref).max() <= 1e-12
    assert np.abs(oracle.linear(W, x) - ref).max() / np.abs(ref).max() < 1e-5
    # one-hot token picks a column
    e = np.zeros((1, K), np.float32); e[0, 77] = 1.0
    assert np.array_equal(oracle.linear(W, e)[0], W[:, 77])
    # identity weight
    I = np.eye(K, dtype=np.float32)
    assert np.array_equal(oracle.linear(I, x), x)
    # all-ones: K * c exactly (c a power of two)
    assert np.all(oracle.linear(np.ones((3, K), np.float32), np.full((1, K), 0.25, np.float32)) == K * 0.25)


def test_quantize_recipe_golden(oracle):
    g = np.load(os.path.join(GOLDEN, "quant.npz"))
    q, s = oracle.quantize_rowscale(g["W"])
    assert np.array_equal(q, g["q"])
    assert np.array_equal(s, g["s"])


def test_int8_exact_with_integer_inputs(oracle):
    N, K = 24, 256
    q = oracle.int8_uniform((N, K), 8)
    s = np.ldexp(1.0, -np.arange(N) % 7).astype(np.float32)
    x = oracle.int8_uniform((2, K), 9, -8, 8).astype(np.float32)
    exact = (x.astype(np.int64) @ q.astype(np.int64).T) * s.astype(np.float64)
    assert np.array_equal(oracle.linear_int8(q, s, x), exact.astype(np.float32))
    assert np.array_equal(oracle.linear_int8_f64(q, s, x), exact)


def test_int8_general_vs_fp64(oracle):
    N, K = 64, 1024
    q = oracle.int8_uniform((N, K), 10)
    s = oracle.uniform(N, 11, 1e-3, 2e-2)
    x = oracle.normal((3, K), 12)
    ref = (x.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)
    assert np.abs(oracle.linear_int8(q, s, x) - ref).max() / np.abs(ref).max() < 1e-5


# ---- norms -----------------------------------------------------------------
def test_rmsnorm_closed_forms(oracle):
    K, eps = 1024, 1e-6
    # reference unit test (tests/unit/test_rmsnorm.cu:54-115): all-ones input,
    # unit effective weight -> 1/sqrt(1+eps); with the (1+w) form that is w=0
    y = oracle.rmsnorm(np.ones((8, K), np.float32), np.zeros(K, np.float32), eps)
    assert np.abs(y - 1.0 / np.sqrt(1.0 + eps)).max() < 1e-6
    c = 3.0
    w = oracle.normal(K, 13, 0.0, 0.02)
    y = oracle.rmsnorm(np.full((1, K), c, np.float32), w, eps)[0]
    exp = c / np.sqrt(c * c + eps) * (1.0 + w.astype(np.float64))
    assert np.abs(y - exp).max() < 1e-6


def test_rmsnorm_vs_fp64(oracle):
    K = 1024
    x = oracle.normal((5, K), 14)
    w = oracle.normal(K, 15, 0.0, 0.02)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-6) * (1.0 + w.astype(np.float64))
    assert np.abs(oracle.rmsnorm_f64(x, w) - ref).max() < 1e-12
    assert np.abs(oracle.rmsnorm(x, w) - ref).max() < 1e-5


def test_residual_rmsnorm(oracle):
    K = 1024
    r = oracle.normal((3, K), 16)
    a = oracle.normal((3, K), 17)
    w = oracle.normal(K, 18, 0.0, 0.02)
    ro, no = oracle.residual_rmsnorm(r, a, w)
    assert np.array_equal(ro, r + a)
    assert np.array_equal(no, oracle.rmsnorm(r + a, w))


# ---- MLP -------------------------------------------------------------------
def test_mlp_matches_reference_golden(oracle):
    g = np.load(os.path.join(GOLDEN, "ref_ops.npz"))
    y = oracle.mlp(g["mlp_Wg"], g["mlp_Wu"], g["mlp_Wd"], g["mlp_x"])
    assert np.array_equal(y, g["mlp_y"])


def test_mlp_vs_numpy_fp64(oracle):
    H, I = 128, 320
    Wg = oracle.normal((I, H), 19, 0.0, 0.05)
    Wu = oracle.normal((I, H), 20, 0.0, 0.05)
    Wd = oracle.normal((H, I), 21, 0.0, 0.05)
    x = oracle.normal((3, H), 22)
    gate = x.astype(np.float64) @ Wg.astype(np.float64).T
    up = x.astype(np.float64) @ Wu.astype(np.float64).T
    ref = (np_silu(gate) * up) @ Wd.astype(np.float64).T
    assert np.abs(oracle.mlp_f64(Wg, Wu, Wd, x) - ref).max() < 1e-12
    assert np.abs(oracle.mlp(Wg, Wu, Wd, x) - ref).max() / np.abs(ref).max() < 1e-5
    # block: x + MLP(RMSNorm(x))
    gm = oracle.normal(H, 23, 0.0, 0.02)
    xd = x.astype(np.float64)
    n = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-6) * (1.0 + gm.astype(np.float64))
    blk = xd + (np_silu(n @ Wg.astype(np.float64).T) * (n @ Wu.astype(np.float64).T)) @ Wd.astype(np.float64).T
    assert np.abs(oracle.mlp_block_f64(Wg, Wu, Wd, gm, x) - blk).max() < 1e-10
    assert np.abs(oracle.mlp_block(Wg, Wu, Wd, gm, x) - blk).max() / np.abs(blk).max() < 1e-5


def test_silu_closed_forms(oracle):
    assert oracle.silu(0.0) == 0.0
    assert abs(oracle.silu(1.0) - 1.0 / (1.0 + np.exp(-1.0))) < 1e-7
    assert abs(oracle.silu(-30.0)) < 1e-11
    assert oracle.silu(30.0) == pytest.approx(30.0, rel=1e-7)


def test_split_q_gate_indices(oracle):
    heads, hd = 8, 256
    raw = np.arange(2 * heads * hd * 2, dtype=np.float32).reshape(2, -1)
    q, g = oracle.split_q_gate(raw, heads, hd)
    r4 = raw.reshape(2, heads, 2, hd)
    assert np.array_equal(q, r4[:, :, 0].reshape(2, -1))
    assert np.array_equal(g, r4[:, :, 1].reshape(2, -1))


# ---- argmax / lm_head ------------------------------------------------------
def test_argmax_matches_reference_sampler(oracle):
    g = np.load(os.path.join(GOLDEN, "ref_ops.npz"))
    ids = [oracle.argmax_first(row) for row in g["greedy_logits"]]
    assert ids == list(g["greedy_ids"])


def test_lmhead_argmax_forms(oracle):
    V, K, M = 3000, 256, 4
    E = oracle.normal((V, K), 24, 0.0, 0.02)
    h = oracle.normal((M, K), 25)
    ids, mx = oracle.lmhead_argmax(E, h)
    logits = h.astype(np.float64) @ E.astype(np.float64).T
    top2 = np.sort(logits, axis=1)[:, -2:]
    for m in range(M):
        if top2[m, 1] - top2[m, 0] > 1e-4:
            assert ids[m] == int(np.argmax(logits[m]))
    assert np.array_equal(ids, [oracle.argmax_first(r) for r in oracle.linear(E, h)])
    # planted ties: identical rows -> lowest index
    E2 = E.copy(); E2[[5, 2000, 2999]] = 0.5
    ids2, _ = oracle.lmhead_argmax(E2, np.abs(h))
    assert np.all(ids2 == 5)
    # bf16 / int8 forms agree with the FP32 form on the rounded / dequantized weight
    Eb, hb = oracle.to_bf16(E), oracle.to_bf16(h)
    ib, mb = oracle.lmhead_argmax_bf16(Eb, hb)
    i32, m32 = oracle.lmhead_argmax(oracle.from_bf16(Eb), oracle.from_bf16(hb))
    assert np.array_equal(ib, i32) and np.array_equal(mb, m32)
    q, s = oracle.quantize_rowscale(E)
    iq, mq = oracle.lmhead_argmax_int8(q, s, h)
    lq = oracle.linear_int8(q, s, h)
    assert np.array_equal(iq, [oracle.argmax_first(r) for r in lq])
    assert np.array_equal(mq, lq.max(axis=1))


# ---- oracle vs the reference's own operators at random shapes ---------------
def _ref_or_skip(oracle):
    R = oracle.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return R


@pytest.mark.parametrize("M,N,K", [(1, 64, 1024), (3, 130, 448)])
def test_linear_vs_ref_lib(oracle, M, N, K):
    R = _ref_or_skip(oracle)
    W = oracle.normal((N, K), 40 + M, 0.0, 0.02)
    x = oracle.normal((M, K), 50 + M)
    y = np.empty((M, N), np.float32)
    assert R.ref_linear(W, x, y, M, N, K) == 0
    assert np.array_equal(oracle.linear(W, x), y)


def test_mlp_vs_ref_lib(oracle):
    R = _ref_or_skip(oracle)
    M, H, I = 2, 128, 384
    Wg = oracle.normal((I, H), 60, 0.0, 0.05)
    Wu = oracle.normal((I, H), 61, 0.0, 0.05)
    Wd = oracle.normal((H, I), 62, 0.0, 0.05)
    x = oracle.normal((M, H), 63)
    y = np.empty((M, H), np.float32)
    assert R.ref_mlp(Wg, Wu, Wd, x, y, M, H, I) == 0
    assert np.array_equal(oracle.mlp(Wg, Wu, Wd, x), y)


def test_greedy_vs_ref_lib(oracle):
    R = _ref_or_skip(oracle)
    for seed in range(5):
        v = oracle.normal(5000, 70 + seed)
        v[[seed * 7, 4000]] = 10.0
        assert oracle.argmax_first(v) == R.ref_greedy(v, v.size) == seed * 7


# ---------------------------------------------------------------------------
# Gated-DeltaNet decode step (language_linear_attn.cpp:143-256)
# ---------------------------------------------------------------------------
def gdn_f64(mixed, a, b, z, conv_w, A_log, dt_bias, norm_w, conv_state, rec_state, nh, kd, vd):
    """Independent float64 restatement in matrix form (einsum per head), for
    one token of each sequence: catches transposed state indices, a wrong
    conv tap order or a missing gate -- the loop-order restatement in
    qw_oracle.c shares none of this code."""
    mixed, a, b, z = (np.atleast_2d(np.asarray(t, np.float64)) for t in (mixed, a, b, z))
    B = mixed.shape[0]
    K = conv_w.shape[1]
    cs = np.asarray(conv_state, np.float64).reshape(B, -1, K - 1).copy()
    rs = np.asarray(rec_state, np.float64).reshape(B, nh, kd, vd).copy()
    w = np.asarray(conv_w, np.float64)
    pre = w[:, K - 1][None, :] * mixed + np.einsum("dj,bdj->bd", w[:, :K - 1], cs)
    co = pre / (1.0 + np.exp(-pre))
    cs = np.concatenate([mixed[:, :, None], cs[:, :, :K - 2]], axis=2) if K > 1 else cs
    q = co[:, :nh * kd].reshape(B, nh, kd)
    k = co[:, nh * kd:2 * nh * kd].reshape(B, nh, kd)
    v = co[:, 2 * nh * kd:].reshape(B, nh, vd)
    q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) / np.sqrt(kd)
    k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    beta = 1.0 / (1.0 + np.exp(-b))
    sp = np.log1p(np.exp(a + np.asarray(dt_bias, np.float64)))
    g = -np.exp(np.asarray(A_log, np.float64)) * sp                     # [B][nh]
    rs = rs * np.exp(g)[:, :, None, None]
    kvm = np.einsum("bhkv,bhk->bhv", rs, k)
    rs = rs + np.einsum("bhk,bhv->bhkv", k, (v - kvm) * beta[:, :, None])
    o = np.einsum("bhkv,bhk->bhv", rs, q)
    o = o / np.sqrt((o * o).mean(-1, keepdims=True) + 1e-6) * np.asarray(norm_w, np.float64)
    o = o.reshape(B, nh * vd) * (z / (1.0 + np.exp(-z)))
    return o, cs, rs.reshape(B, nh, kd * vd)


def _gdn_case(oracle, B, nh, kd, vd, K, seed):
    cd = 2 * nh * kd + nh * vd
    return dict(mixed=oracle.normal((B, cd), seed), a=oracle.normal((B, nh), seed + 1),
                b=oracle.normal((B, nh), seed + 2), z=oracle.normal((B, nh * vd), seed + 3),
                conv_w=oracle.normal((cd, K), seed + 4, 0.0, 0.5), A_log=oracle.normal((nh,), seed + 5, 0.0, 0.5),
                dt_bias=oracle.normal((nh,), seed + 6, 0.0, 0.5), norm_w=1.0 + oracle.normal((vd,), seed + 7, 0.0, 0.1),
                conv_state=oracle.normal((B, cd, K - 1), seed + 8), rec_state=oracle.normal((B, nh, kd * vd), seed + 9, 0.0, 0.3))


def test_gdn_matches_reference_golden(oracle):
    """Projections (oracle linear) + the step + out projection reproduce the
    reference's own LinearAttention::forward bit for bit over 3 tokens,
    including both updated states (tests/golden/ref_ops.npz)."""
    g = np.load(os.path.join(GOLDEN, "ref_ops.npz"))
    nh, kd, vd = 2, 8, 8
    cs, rs = g["gdn_conv_state"], g["gdn_rec_state"]
    ys = []
    for t in range(g["gdn_x"].shape[0]):
        x = g["gdn_x"][t:t + 1]
        mixed, a, b, z = (oracle.linear(g[n], x) for n in ("gdn_Wqkv", "gdn_Wa", "gdn_Wb", "gdn_Wz"))
        o, cs, rs = oracle.gdn_step(mixed, a, b, z, g["gdn_conv_w"], g["gdn_A_log"], g["gdn_dt_bias"],
                                    g["gdn_norm_w"], cs, rs, nh, kd, vd)
        ys.append(oracle.linear(g["gdn_Wout"], o))
    assert np.array_equal(np.concatenate(ys), g["gdn_y"])
    assert np.array_equal(cs, g["gdn_conv_state_out"])
    assert np.array_equal(rs.reshape(g["gdn_rec_state_out"].shape), g["gdn_rec_state_out"])


def test_gdn_vs_ref_lib(oracle):
    """Live reference build, Qwen3.5-0.8B head shape (nh 16, kd = vd = 128)."""
    if oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    H, nh, kd, vd, K, T = 256, 16, 128, 128, 4, 2
    cd = 2 * nh * kd + nh * vd
    W = {n: oracle.normal(sh, 60 + i, 0.0, 0.05) for i, (n, sh) in enumerate(
        [("Wqkv", (cd, H)), ("Wa", (nh, H)), ("Wb", (nh, H)), ("Wz", (nh * vd, H)), ("Wout", (H, nh * vd))])}
    c = _gdn_case(oracle, 1, nh, kd, vd, K, 70)
    x = oracle.normal((T, H), 80)
    y_ref, cs_ref, rs_ref = oracle.ref_linear_attn(x, W["Wqkv"], W["Wa"], W["Wb"], W["Wz"], c["conv_w"], c["A_log"],
                                                   c["dt_bias"], c["norm_w"], W["Wout"], c["conv_state"][0],
                                                   c["rec_state"][0], nh, kd, vd)
    cs, rs = c["conv_state"], c["rec_state"]
    for t in range(T):
        xt = x[t:t + 1]
        o, cs, rs = oracle.gdn_step(oracle.linear(W["Wqkv"], xt), oracle.linear(W["Wa"], xt),
                                    oracle.linear(W["Wb"], xt), oracle.linear(W["Wz"], xt), c["conv_w"],
                                    c["A_log"], c["dt_bias"], c["norm_w"], cs, rs, nh, kd, vd)
        assert np.array_equal(oracle.linear(W["Wout"], o)[0], y_ref[t])
    assert np.array_equal(cs[0], cs_ref) and np.array_equal(rs[0], rs_ref)


@pytest.mark.parametrize("B,nh,kd,vd,K", [(1, 2, 8, 8, 4), (3, 4, 16, 8, 4), (2, 16, 128, 128, 4), (2, 2, 8, 8, 2)])
def test_gdn_vs_float64_matrix_form(oracle, relerr, B, nh, kd, vd, K):
    c = _gdn_case(oracle, B, nh, kd, vd, K, 90 + K)
    cs, rs, cs64, rs64 = c["conv_state"], c["rec_state"], c["conv_state"], c["rec_state"]
    for step in range(3):
        mixed = oracle.normal(c["mixed"].shape, 100 + step)
        o, cs, rs = oracle.gdn_step(mixed, c["a"], c["b"], c["z"], c["conv_w"], c["A_log"], c["dt_bias"],
                                    c["norm_w"], cs, rs, nh, kd, vd)
        o64, cs64, rs64 = gdn_f64(mixed, c["a"], c["b"], c["z"], c["conv_w"], c["A_log"], c["dt_bias"],
                                  c["norm_w"], cs64, rs64, nh, kd, vd)
        assert relerr(o, o64) <= 1e-5
        assert relerr(rs.reshape(rs64.shape), rs64) <= 1e-5
        assert np.array_equal(cs.reshape(cs64.shape), cs64.astype(np.float32))   # pure copies


def test_gdn_closed_forms(oracle):
    """beta -> 0 (b = -80): the state only decays, S' = exp(g) S, and o is
    S'^T q; a single last conv tap of 1: the conv output is silu(x)."""
    B, nh, kd, vd, K = 1, 2, 8, 8, 4
    c = _gdn_case(oracle, B, nh, kd, vd, K, 120)
    c["b"][:] = -80.0
    c["conv_w"][:] = 0.0
    c["conv_w"][:, K - 1] = 1.0
    c["norm_w"][:] = 1.0
    c["z"][:] = 40.0                                   # silu(z) = z
    o, cs, rs = oracle.gdn_step(c["mixed"], c["a"], c["b"], c["z"], c["conv_w"], c["A_log"], c["dt_bias"],
                                c["norm_w"], c["conv_state"], c["rec_state"], nh, kd, vd)
    x = c["mixed"][0].astype(np.float64)
    co = x / (1 + np.exp(-x))
    q = co[:nh * kd].reshape(nh, kd)
    q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) / np.sqrt(kd)
    g = -np.exp(c["A_log"].astype(np.float64)) * np.log1p(np.exp(c["a"][0] + c["dt_bias"]))
    S = c["rec_state"][0].reshape(nh, kd, vd).astype(np.float64) * np.exp(g)[:, None, None]
    np.testing.assert_allclose(rs[0].reshape(nh, kd, vd), S, rtol=1e-5, atol=1e-7)
    oo = np.einsum("hkv,hk->hv", S, q)
    oo = oo / np.sqrt((oo * oo).mean(-1, keepdims=True) + 1e-6) * 40.0
    np.testing.assert_allclose(o[0].reshape(nh, vd), oo, rtol=1e-4, atol=1e-5)
    # conv state: newest first, the oldest tap dropped
    assert np.array_equal(cs[0][:, 0], c["mixed"][0])
    assert np.array_equal(cs[0][:, 1:], c["conv_state"][0][:, :K - 2])


# ---- gated full attention ------------------------------------------------------
def _split_qg(qraw, nh, hd):
    """The per-head Q/gate interleave of the reference (language_full_attn.cpp:133-140)."""
    r = qraw.reshape(qraw.shape[0], nh, 2, hd)
    return np.ascontiguousarray(r[:, :, 0].reshape(qraw.shape[0], -1)), \
        np.ascontiguousarray(r[:, :, 1].reshape(qraw.shape[0], -1))


def test_full_attn_matches_reference_golden(oracle):
    """Projections (oracle linear) + norm/RoPE/cache/attention/gate + o_proj
    reproduce the reference's own FullAttention::forward bit for bit over 6
    tokens from an empty cache (tests/golden/ref_ops.npz; theta 100)."""
    g = np.load(os.path.join(GOLDEN, "ref_ops.npz"))
    nh, nkv, hd = 4, 2, 16
    x = g["fa_x"]
    q, gate = _split_qg(oracle.linear(g["fa_Wq"], x), nh, hd)
    k, v = oracle.linear(g["fa_Wk"], x), oracle.linear(g["fa_Wv"], x)
    out, _ = oracle.full_attn_seq(q, gate, k, v, g["fa_qn"], g["fa_kn"], nh, nkv, hd, rotary_dim=4, theta=100.0)
    assert np.array_equal(oracle.linear(g["fa_Wo"], out), g["fa_y"])


def test_full_attn_vs_ref_lib(oracle):
    """Live reference build at the Qwen3.5-0.8B shape (8 heads, 2 KV heads,
    head dim 256, rotary 64, theta 1e7), 3 tokens."""
    if oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    H, nh, nkv, hd, T = 128, 8, 2, 256, 3
    Wq = oracle.normal((nh * hd * 2, H), 130, 0.0, 0.05)
    Wk, Wv = oracle.normal((nkv * hd, H), 131, 0.0, 0.05), oracle.normal((nkv * hd, H), 132, 0.0, 0.05)
    qn, kn = oracle.normal((hd,), 133, 0.0, 0.1), oracle.normal((hd,), 134, 0.0, 0.1)
    Wo = oracle.normal((H, nh * hd), 135, 0.0, 0.05)
    x = oracle.normal((T, H), 136)
    y_ref = oracle.ref_full_attn(x, Wq, Wk, Wv, qn, kn, Wo, nh, nkv, hd, hd)
    q, gate = _split_qg(oracle.linear(Wq, x), nh, hd)
    out, _ = oracle.full_attn_seq(q, gate, oracle.linear(Wk, x), oracle.linear(Wv, x), qn, kn, nh, nkv, hd)
    assert np.array_equal(oracle.linear(Wo, out), y_ref)


def full_attn_f64(q, gate, k, v, qn, kn, nh, nkv, hd, rotary_dim, theta):
    """numpy float64 statement of the same T tokens from an empty cache."""
    T = q.shape[0]
    q = q.astype(np.float64).reshape(T, nh, hd)
    k = k.astype(np.float64).reshape(T, nkv, hd)
    v = v.astype(np.float64).reshape(T, nkv, hd)
    q = q / np.sqrt((q * q).mean(-1, keepdims=True) + 1e-6) * (1.0 + qn)
    k = k / np.sqrt((k * k).mean(-1, keepdims=True) + 1e-6) * (1.0 + kn)
    d = np.arange(0, rotary_dim, 2)
    ang = np.arange(T)[:, None] * (1.0 / theta ** (d / rotary_dim))[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    for x in (q, k):
        x0, x1 = x[..., d].copy(), x[..., d + 1].copy()
        x[..., d], x[..., d + 1] = x0 * c - x1 * s, x0 * s + x1 * c
    out = np.zeros((T, nh, hd))
    for t in range(T):
        for h in range(nh):
            g = h // (nh // nkv)
            sc = k[:t + 1, g] @ q[t, h] / np.sqrt(hd)
            w = np.exp(sc - sc.max())
            w /= w.sum()
            out[t, h] = (w @ v[:t + 1, g]) / (1.0 + np.exp(-gate.reshape(T, nh, hd)[t, h]))
    return out.reshape(T, -1)


def test_full_attn_vs_float64(oracle, relerr):
    nh, nkv, hd, T = 8, 2, 256, 7
    q, gate = oracle.normal((T, nh * hd), 140), oracle.normal((T, nh * hd), 141)
    k, v = oracle.normal((T, nkv * hd), 142), oracle.normal((T, nkv * hd), 143)
    qn, kn = oracle.normal((hd,), 144, 0.0, 0.1), oracle.normal((hd,), 145, 0.0, 0.1)
    out, _ = oracle.full_attn_seq(q, gate, k, v, qn, kn, nh, nkv, hd, rotary_dim=64, theta=1000.0)
    ref = full_attn_f64(q, gate, k, v, qn, kn, nh, nkv, hd, 64, 1000.0)
    assert relerr(out, ref) <= 1e-5


def test_full_attn_closed_forms(oracle):
    """Position 0 leaves q, k unrotated; the first token attends only to itself,
    so its output is v * sigmoid(gate) whatever q and k are; a constant input
    normalizes to (1 + w)."""
    nh, nkv, hd = 4, 2, 16
    q, k = oracle.normal(nh * hd, 150), oracle.normal(nkv * hd, 151)
    w0 = np.zeros(hd, np.float32)
    q1, k1 = oracle.attn_norm_rope(q, k, w0, w0, 0, nh, nkv, hd, 8, 1.0e4)
    qr = q.reshape(nh, hd).astype(np.float64)
    np.testing.assert_allclose(q1.reshape(nh, hd), qr / np.sqrt((qr * qr).mean(-1, keepdims=True) + 1e-6),
                               rtol=1e-6, atol=1e-6)
    const = np.full(nh * hd, 3.0, np.float32)
    w = oracle.normal(hd, 152, 0.0, 0.1)
    qc, _ = oracle.attn_norm_rope(const, np.full(nkv * hd, 3.0, np.float32), w, w, 0, nh, nkv, hd, 8, 1.0e4)
    np.testing.assert_allclose(qc.reshape(nh, hd), np.tile(3.0 / np.sqrt(9.0 + 1e-6) * (1.0 + w), (nh, 1)),
                               rtol=1e-6)
    gate, v = oracle.normal((1, nh * hd), 153), oracle.normal((1, nkv * hd), 154)
    out, _ = oracle.full_attn_seq(q[None], gate, k[None], v, w0, w0, nh, nkv, hd, rotary_dim=8)
    vv = v.reshape(nkv, hd)[np.arange(nh) // 2].reshape(-1)
    np.testing.assert_allclose(out[0], vv / (1.0 + np.exp(-gate[0].astype(np.float64))), rtol=1e-6, atol=1e-7)
    # RoPE is a rotation: each rotated pair keeps its norm (position 5, unit norm weights)
    q5, _ = oracle.attn_norm_rope(q, k, w0, w0, 5, nh, nkv, hd, 8, 1.0)
    n0 = q1.reshape(nh, hd // 2, 2)[:, :4]
    n5 = q5.reshape(nh, hd // 2, 2)[:, :4]
    np.testing.assert_allclose((n5 ** 2).sum(-1), (n0 ** 2).sum(-1), rtol=1e-5)
    assert np.array_equal(q5.reshape(nh, hd)[:, 8:], q1.reshape(nh, hd)[:, 8:])


def test_kv_quant_int8_hand_worked(oracle):
    """The INT8 KV recipe on vectors worked by hand: scale = max|x|/127, ties
    of x/scale round away from zero, the maximum maps to +-127, an all-zero
    (or tiny) head gets scale 1."""
    x = np.zeros(8, np.float32)
    x[:5] = [127.0, -63.5, 2.5, -0.5, 1.49]   # scale exactly 1.0
    q, s = oracle.kv_quant_int8(x)
    assert s == 1.0 and list(q) == [127, -64, 3, -1, 1, 0, 0, 0]
    q, s = oracle.kv_quant_int8(np.array([0.0, -254.0, 1.0, 3.0], np.float32))   # scale 2
    assert s == 2.0 and list(q) == [0, -127, 1, 2]                                # 0.5 -> 1, 1.5 -> 2
    q, s = oracle.kv_quant_int8(np.zeros(4, np.float32))
    assert s == 1.0 and not q.any()
    q, s = oracle.kv_quant_int8(np.array([1e-7, -1e-7], np.float32))             # max/127 < 1e-8
    assert s == 1.0 and not q.any()


def test_full_attn_int8_cache_reads_each_token_scale(oracle, relerr):
    """The INT8 cache keeps per-(token, head) scales and the oracle reads each
    token back with its own: with tokens of very different magnitudes the
    result stays within INT8 rounding of the FP32-cache result."""
    nh, nkv, hd, T = 8, 2, 256, 5
    q, gate = oracle.normal((T, nh * hd), 160), oracle.normal((T, nh * hd), 161)
    k = oracle.normal((T, nkv * hd), 162)
    v = oracle.normal((T, nkv * hd), 163) * np.array([1, 100, 0.01, 10, 1], np.float32)[:, None]
    qn = kn = np.zeros(hd, np.float32)
    o32, _ = oracle.full_attn_seq(q, gate, k, v, qn, kn, nh, nkv, hd)
    o8, (kc, vc, ks, vs) = oracle.full_attn_seq(q, gate, k, v, qn, kn, nh, nkv, hd, int8=True)
    assert relerr(o8, o32) <= 2e-2
    assert ks.shape == (T, nkv) and len(set(np.round(vs[:, 0], 6))) == T
