"""GPU parity of the projection kernels (qw_linear, qw_weight_pack) against the
CPU oracle.

Bars (written next to each check):
  * packing: bit-exact (BF16 bits, INT8 values and scales vs the oracle's
    restatement of mlp_cuda.cu:22-39);
  * FP32 weights x FP32 activations: <= 1e-5 normwise vs FP64;
  * products on the exact stored operands (bf16/int8 weights, the activation
    as stored): <= 2e-5 normwise vs FP64 for FP32 outputs (catches any
    dropped/misplaced term: one wrong k is an O(1/sqrt(K)) error);
  * BF16 paths <= 1e-2 vs FP64 on the unrounded FP32 weights,
    INT8 paths <= 1e-3 vs the reference's dequant-then-matmul.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


XDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def stored_x(x, name):
    """The activation values the GPU actually sees (rounded to its dtype)."""
    return host(dev(x, XDT[name]))


# ----------------------------------------------------------------------------
# packing
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(40, 128), (16, 64), (3584, 1024)])
def test_pack_roundtrip(qw, ctx, oracle, N, K):
    W = oracle.normal((N, K), 11, 0.0, 0.02)
    w32 = qw.Weight.pack(ctx, W, qw.WFMT_F32)
    got, _ = w32.unpack()
    assert np.array_equal(got, W)
    wbf = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    got, _ = wbf.unpack()
    assert np.array_equal(got, oracle.to_bf16(W))          # bit-exact RNE
    wi8 = qw.Weight.pack(ctx, W, qw.WFMT_INT8)
    q, s = wi8.unpack()
    q_ref, s_ref = oracle.quantize_rowscale(W)
    assert np.array_equal(s, s_ref)                          # bit-exact scales
    assert np.array_equal(q, q_ref)                          # bit-exact codes


def test_pack_int8_edge_rows(qw, ctx, oracle):
    """Zero row (scale 1.0), a row whose max is tiny (<= 1e-8*127), exact
    .5 ties (roundf rounds half away from zero), and +-max clamping."""
    K = 64
    W = np.zeros((4, K), np.float32)
    W[1, :] = 1e-9
    W[2, :] = np.linspace(-127, 127, K).astype(np.float32)
    W[2, 0] = 2.5; W[2, 1] = -2.5; W[2, 2] = 0.5; W[2, 3] = -0.5
    W[3, :] = oracle.normal((K,), 5, 0.0, 3.0)
    q, s = qw.Weight.pack(ctx, W, qw.WFMT_INT8).unpack()
    q_ref, s_ref = oracle.quantize_rowscale(W)
    assert s[0] == 1.0 and s[1] == 1.0
    assert np.array_equal(q, q_ref) and np.array_equal(s, s_ref)
    assert q[2, 0] == 3 and q[2, 1] == -3 and q[2, 2] == 1 and q[2, 3] == -1


def test_pack_prequantized(qw, ctx, oracle):
    N, K = 48, 192
    q = oracle.int8_uniform((N, K), 3)
    s = oracle.uniform((N,), 4, 1e-3, 2e-2)
    q2, s2 = qw.Weight.pack(ctx, q, qw.WFMT_INT8, scales=s).unpack()
    assert np.array_equal(q2, q) and np.array_equal(s2, s)


def test_pack_glu_roundtrip(qw, ctx, oracle):
    N, K = 48, 128
    G = oracle.normal((N, K), 1, 0.0, 0.02)
    U = oracle.normal((N, K), 2, 0.0, 0.02)
    w = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_INT8)
    q, s = w.unpack()
    qg, sg = oracle.quantize_rowscale(G)
    qu, su = oracle.quantize_rowscale(U)
    assert np.array_equal(q[:N], qg) and np.array_equal(q[N:], qu)
    assert np.array_equal(s[:N], sg) and np.array_equal(s[N:], su)


# ----------------------------------------------------------------------------
# closed forms: these fail for a transposed operand or a wrong k permutation
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", ["f32", "bf16", "int8"])
def test_identity_and_onehot(qw, ctx, oracle, fmt):
    K = 128
    f = {"f32": qw.WFMT_F32, "bf16": qw.WFMT_BF16, "int8": qw.WFMT_INT8}[fmt]
    W = np.eye(K, dtype=np.float32)
    w = qw.Weight.pack(ctx, W, f)
    x = np.round(oracle.normal((3, K), 7) * 8) / 8          # exact in bf16/f16
    xt = dev(x, torch.float32)
    y = torch.empty(3, K, device="cuda")
    qw.linear(ctx, w, xt, y)
    torch.cuda.synchronize()
    if fmt == "int8":                                        # q = 127*I, s = 1/127
        q, s = w.unpack()
        assert np.array_equal(host(y), (x * np.float32(127)) * s[None, :])
    else:
        assert np.array_equal(host(y), x)                    # W = I  =>  y = x
    # one-hot x picks a column of W
    N = 80
    W2 = np.round(oracle.normal((N, K), 8) * 64) / 64
    w2 = qw.Weight.pack(ctx, W2, f)
    scale = w2.unpack()[1]
    for k in (0, 1, 7, 8, 31, 32, 63, 64, 127):
        e = np.zeros((1, K), np.float32)
        e[0, k] = 1.0
        y2 = torch.empty(1, N, device="cuda")
        qw.linear(ctx, w2, dev(e), y2)
        torch.cuda.synchronize()
        if fmt == "int8":
            qcol = w2.unpack()[0][:, k].astype(np.float32) * scale
            assert np.array_equal(host(y2)[0], qcol)
        else:
            assert np.array_equal(host(y2)[0], W2[:, k])


# ----------------------------------------------------------------------------
# parity on random inputs
# ----------------------------------------------------------------------------

SHAPES = [(3584, 1024), (1024, 3584), (40, 128), (16, 1024)]


def _exact_ref(oracle, fmt, W, wobj, xs):
    """FP64 product on the exact operands the GPU uses."""
    if fmt == "int8":
        q, s = wobj.unpack()
        return oracle.linear_int8_f64(q, s, xs)
    if fmt == "bf16":
        return oracle.linear_f64(oracle.round_bf16(W), xs)
    return oracle.linear_f64(W, xs)


@pytest.mark.parametrize("fmt,xname", [
    ("f32", "f32"), ("f32", "bf16"),
    ("bf16", "bf16"), ("bf16", "f32"), ("bf16", "f16"),
    ("int8", "f16"), ("int8", "bf16"), ("int8", "f32"),
])
@pytest.mark.parametrize("M", [1, 7, 16, 32, 45, 100])
def test_linear_parity(qw, ctx, oracle, relerr, fmt, xname, M):
    f = {"f32": qw.WFMT_F32, "bf16": qw.WFMT_BF16, "int8": qw.WFMT_INT8}[fmt]
    for si, (N, K) in enumerate(SHAPES):
        if M > 16 and si == 0 and fmt == "f32":
            continue  # keep the FP64 reference cheap
        W = oracle.normal((N, K), 100 + si, 0.0, 0.02)
        x = oracle.normal((M, K), 200 + si + M)
        w = qw.Weight.pack(ctx, W, f)
        xt = dev(x, XDT[xname])
        y = torch.empty(M, N, device="cuda")
        qw.linear(ctx, w, xt, y)
        torch.cuda.synchronize()
        got = host(y)
        xs = stored_x(x, xname)
        ref = _exact_ref(oracle, fmt, W, w, xs)
        # exact operands: only FP32 accumulation error remains, except for the
        # hi/lo bf16 split of an FP32 activation (16 of its 24 bits kept)
        tol = 1e-4 if (fmt == "bf16" and xname == "f32") else 2e-5
        assert relerr(got, ref) <= tol, (N, K, M, relerr(got, ref))
        # north-star bars
        if fmt == "bf16":
            assert relerr(got, oracle.linear_f64(W, xs)) <= 1e-2
        if fmt == "int8":
            q, s = w.unpack()
            assert relerr(got, oracle.linear_int8(q, s, xs)) <= 1e-3
        if fmt == "f32" and xname == "f32":
            assert relerr(got, oracle.linear_f64(W, x)) <= 1e-5


@pytest.mark.parametrize("ydt", ["bf16", "f16"])
def test_linear_output_dtypes(qw, ctx, oracle, relerr, ydt):
    N, K, M = 1024, 2048, 4
    W = oracle.normal((N, K), 31, 0.0, 0.02)
    x = oracle.normal((M, K), 32)
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    y = torch.empty(M, N, device="cuda", dtype=XDT[ydt])
    qw.linear(ctx, w, dev(x, torch.bfloat16), y)
    torch.cuda.synchronize()
    ref = oracle.linear_f64(oracle.round_bf16(W), stored_x(x, "bf16"))
    assert relerr(host(y), ref) <= 4e-3                     # one output rounding


def test_linear_deterministic(qw, ctx, oracle):
    """Split-K partials are summed in split order: bitwise repeatable."""
    N, K, M = 1024, 3584, 3
    w = qw.Weight.pack(ctx, oracle.normal((N, K), 41, 0.0, 0.02), qw.WFMT_BF16)
    x = dev(oracle.normal((M, K), 42), torch.bfloat16)
    outs = []
    for _ in range(3):
        y = torch.empty(M, N, device="cuda")
        qw.linear(ctx, w, x, y)
        torch.cuda.synchronize()
        outs.append(host(y))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])


# ----------------------------------------------------------------------------
# epilogues
# ----------------------------------------------------------------------------

@pytest.mark.parametrize("M", [1, 20, 50])
@pytest.mark.parametrize("rdt", ["f32", "bf16"])
def test_residual_epilogue(qw, ctx, oracle, relerr, M, rdt):
    N, K = 1024, 2048                                        # out-proj shape
    W = oracle.normal((N, K), 51, 0.0, 0.02)
    x = oracle.normal((M, K), 52)
    r = oracle.normal((M, N), 53)
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    res = dev(r, XDT[rdt])
    y = res.clone() if rdt == "f32" else torch.empty(M, N, device="cuda")
    # in place when the residual is FP32 (y aliases residual)
    qw.linear(ctx, w, dev(x, torch.bfloat16), y, residual=(y if rdt == "f32" else res))
    torch.cuda.synchronize()
    ref = oracle.linear_f64(oracle.round_bf16(W), stored_x(x, "bf16")) + host(res)
    assert relerr(host(y), ref) <= 2e-5


@pytest.mark.parametrize("fmt", ["bf16", "int8", "f32"])
@pytest.mark.parametrize("M", [1, 9, 32, 70])
def test_norm_prologue(qw, ctx, oracle, relerr, fmt, M):
    """x := RMSNorm(x)*(1+gamma) folded into the projection."""
    N, K = 512, 1024
    f = {"f32": qw.WFMT_F32, "bf16": qw.WFMT_BF16, "int8": qw.WFMT_INT8}[fmt]
    W = oracle.normal((N, K), 61, 0.0, 0.02)
    gamma = oracle.normal((K,), 62, 0.0, 0.02)
    x = oracle.normal((M, K), 63) * 3.0
    w = qw.Weight.pack(ctx, W, f)
    xname = {"bf16": "bf16", "int8": "f16", "f32": "f32"}[fmt]
    xt = dev(x, XDT[xname])
    y = torch.empty(M, N, device="cuda")
    qw.linear(ctx, w, xt, y, gamma=dev(gamma), eps=1e-6)
    torch.cuda.synchronize()
    xs = stored_x(x, xname)
    xn = oracle.rmsnorm_f64(xs, gamma)
    if fmt == "int8":
        q, s = w.unpack()
        ref = (xn @ q.astype(np.float64).T) * s.astype(np.float64)
        bar = 1e-3
    elif fmt == "bf16":
        ref = xn @ oracle.round_bf16(W).astype(np.float64).T
        bar = 1e-2
    else:
        ref = xn @ W.astype(np.float64).T
        bar = 1e-5
    assert relerr(host(y), ref) <= bar


def test_split_q_gate(qw, ctx, oracle):
    """Full-attention q_proj [2*8*256][1024]: per head, rows [h*512, h*512+256)
    are Q and the next 256 the output gate (language_full_attn.cpp:133-140)."""
    heads, D, K, M = 8, 256, 1024, 3
    W = oracle.normal((2 * heads * D, K), 71, 0.0, 0.02)
    x = oracle.normal((M, K), 72)
    w = qw.Weight.pack(ctx, W, qw.WFMT_F32)
    q = torch.empty(M, heads * D, device="cuda")
    g = torch.empty(M, heads * D, device="cuda")
    qw.linear(ctx, w, dev(x), q, y2=g, split_period=D)
    full = torch.empty(M, 2 * heads * D, device="cuda")
    qw.linear(ctx, w, dev(x), full)
    torch.cuda.synchronize()
    q_ref, g_ref = oracle.split_q_gate(host(full), heads, D)
    assert np.array_equal(host(q), q_ref) and np.array_equal(host(g), g_ref)


@pytest.mark.parametrize("fmt", ["bf16", "int8", "f32"])
@pytest.mark.parametrize("M", [1, 16, 24, 80])
def test_glu_silu_mul(qw, ctx, oracle, relerr, fmt, M):
    I, H = 3584, 1024
    f = {"f32": qw.WFMT_F32, "bf16": qw.WFMT_BF16, "int8": qw.WFMT_INT8}[fmt]
    G = oracle.normal((I, H), 81, 0.0, 0.02)
    U = oracle.normal((I, H), 82, 0.0, 0.02)
    x = oracle.normal((M, H), 83)
    w = qw.Weight.pack_glu(ctx, G, U, f)
    xname = {"bf16": "bf16", "int8": "f16", "f32": "f32"}[fmt]
    h = torch.empty(M, I, device="cuda")
    qw.linear(ctx, w, dev(x, XDT[xname]), h)
    torch.cuda.synchronize()
    xs = stored_x(x, xname).astype(np.float64)
    if fmt == "int8":
        q, s = w.unpack()
        g = (xs @ q[:I].astype(np.float64).T) * s[:I]
        u = (xs @ q[I:].astype(np.float64).T) * s[I:]
    elif fmt == "bf16":
        g = xs @ oracle.round_bf16(G).astype(np.float64).T
        u = xs @ oracle.round_bf16(U).astype(np.float64).T
    else:
        g = xs @ G.astype(np.float64).T
        u = xs @ U.astype(np.float64).T
    ref = g / (1.0 + np.exp(-g)) * u
    assert relerr(host(h), ref) <= 1e-4


def test_error_codes(qw, ctx, oracle):
    W = oracle.normal((64, 128), 1, 0.0, 0.02)
    w = qw.Weight.pack(ctx, W, qw.WFMT_BF16)
    x = torch.zeros(2, 128, device="cuda", dtype=torch.bfloat16)
    y = torch.zeros(2, 64, device="cuda")
    with pytest.raises(qw.QwError) as e:
        qw.linear(ctx, w, x[:, 1:], y, ldx=128)             # misaligned x
    assert e.value.status == qw.ERR_ALIGN
    with pytest.raises(qw.QwError) as e:
        qw.Weight.pack(ctx, oracle.normal((8, 100), 1), qw.WFMT_BF16)   # K % 64
    assert e.value.status == qw.ERR_SHAPE
    with pytest.raises(qw.QwError) as e:
        qw.Weight.pack(ctx, oracle.int8_uniform((8, 64), 1), qw.WFMT_INT8)  # no scales
    assert e.value.status == qw.ERR_NULL
    with pytest.raises(qw.QwError) as e:
        qw.linear(ctx, w, x, y, gamma=torch.zeros(128, device="cuda"), eps=0.0)
    assert e.value.status == qw.ERR_INVALID


@pytest.mark.parametrize("fmt", ["bf16", "int8"])
def test_split_k_handoff_repeatable(qw, ctx, oracle, relerr, fmt):
    """Split-K tiles (N=1024 over K=3584 is split across many waves): 200
    back-to-back launches must all equal the first bitwise and the FP64
    reference -- a partial read before its writer finished would show up as
    a missing 1/S of the sum."""
    f = {"bf16": qw.WFMT_BF16, "int8": qw.WFMT_INT8}[fmt]
    N, K, M = 1024, 3584, 2
    W = oracle.normal((N, K), 91, 0.0, 0.02)
    w = qw.Weight.pack(ctx, W, f)
    x = oracle.normal((M, K), 92)
    xt = dev(x, torch.float16 if fmt == "int8" else torch.bfloat16)
    ys = torch.empty(200, M, N, device="cuda")
    for i in range(200):
        qw.linear(ctx, w, xt, ys[i])
    torch.cuda.synchronize()
    got = ys.cpu().numpy()
    assert (got == got[0][None]).all()
    xs = host(xt)
    ref = oracle.linear_int8_f64(*w.unpack(), xs) if fmt == "int8" else oracle.linear_f64(oracle.round_bf16(W), xs)
    assert relerr(got[0], ref) <= 2e-5


@pytest.mark.parametrize("kernel", ["gemv", "skinny"])
@pytest.mark.parametrize("M", [2, 70])
def test_forced_split_k(qw, oracle, relerr, kernel, M):
    """Cross-workgroup split-K (forced with QW_SKINNY_MIN_ITEMS) on both
    small-M kernels, with and without token groups, with the RMSNorm sums of
    squares and a residual riding along: repeated calls bit-identical and
    equal to the FP64 reference (counters and partials of each group and
    tile kept apart and re-armed)."""
    import os
    os.environ["QW_SKINNY_MIN_ITEMS"] = "1024"
    os.environ["QW_GEMV"] = "1" if kernel == "gemv" else "0"
    try:
        c = qw.Context(0)
    finally:
        del os.environ["QW_SKINNY_MIN_ITEMS"]
        del os.environ["QW_GEMV"]
    N, K = 1024, 3584
    W = oracle.normal((N, K), 95, 0.0, 0.02)
    gam = oracle.normal((K,), 96, 0.0, 0.1)
    x = oracle.normal((M, K), 97)
    r = oracle.normal((M, N), 98)
    w = qw.Weight.pack(c, W, qw.WFMT_BF16)
    xt = dev(x, torch.bfloat16)
    rt = dev(r)
    ys = torch.empty(5, M, N, device="cuda")
    for i in range(5):
        qw.linear(c, w, xt, ys[i], residual=rt, gamma=dev(gam) if M <= 16 else None)
    torch.cuda.synchronize()
    got = ys.cpu().numpy()
    assert (got == got[0][None]).all()
    xs = host(xt)
    xin = oracle.rmsnorm_f64(xs, gam) if M <= 16 else xs
    ref = xin @ oracle.round_bf16(W).astype(np.float64).T + r
    assert relerr(got[0], ref) <= (1e-2 if M <= 16 else 2e-5)
    torch.cuda.synchronize()
    c.close()


# ----------------------------------------------------------------------------
# RMSNorm weight folded into the projection (qw_weight_fold_norm)
# ----------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("fmt,M", [("bf16", 1), ("bf16", 8), ("bf16", 16), ("bf16", 40), ("f32", 3)])
def test_fold_norm_linear(qw, ctx, oracle, relerr, fmt, M):
    """W*(1+gamma) with rms-only scaling equals RMSNorm(x)*(1+gamma) then W,
    against the FP64 oracle (GEMV, skinny and GEMM paths by M / dtype)."""
    N, K = 3584, 1024
    W = oracle.normal((N, K), 710, 0.0, 0.02)
    gam = oracle.normal((K,), 711, 0.0, 0.1)
    x = oracle.normal((M, K), 712)
    f = qw.WFMT_BF16 if fmt == "bf16" else qw.WFMT_F32
    xdt = torch.bfloat16 if fmt == "bf16" else torch.float32
    w = qw.Weight.pack(ctx, W, f).fold_norm(torch.from_numpy(gam).cuda())
    xt = torch.from_numpy(x).cuda().to(xdt)
    y = torch.empty(M, N, device="cuda")
    qw.linear(ctx, w, xt, y, norm=True)
    torch.cuda.synchronize()
    xs = xt.float().cpu().numpy()
    ref = oracle.linear_f64(W, oracle.rmsnorm_f64(xs, gam).astype(np.float32))
    assert relerr(y.cpu().numpy(), ref) <= (1e-2 if fmt == "bf16" else 1e-5)


@pytest.mark.gpu
def test_fold_norm_mlp_and_errors(qw, ctx, oracle, relerr):
    H, I, M = 1024, 3584, 2
    G = oracle.normal((I, H), 720, 0.0, 0.02)
    U = oracle.normal((I, H), 721, 0.0, 0.02)
    D = oracle.normal((H, I), 722, 0.0, 0.02)
    gam = oracle.normal((H,), 723, 0.0, 0.1)
    x = oracle.normal((M, H), 724)
    gt = torch.from_numpy(gam).cuda()
    gu = qw.Weight.pack_glu(ctx, G, U, qw.WFMT_BF16).fold_norm(gt)
    dn = qw.Weight.pack(ctx, D, qw.WFMT_BF16)
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    y = torch.empty(M, H, device="cuda")
    qw.mlp_fused(ctx, gu, dn, xt, y, residual=xt)
    torch.cuda.synchronize()
    ref = oracle.mlp_block_f64(G, U, D, gam, xt.float().cpu().numpy())
    assert relerr(y.cpu().numpy(), ref) <= 1e-2
    # gamma given again, folding twice, INT8 weights: refused
    with pytest.raises(qw.QwError) as e:
        qw.mlp_fused(ctx, gu, dn, xt, y, gamma=gt, residual=xt)
    assert e.value.status == qw.ERR_INVALID
    with pytest.raises(qw.QwError) as e:
        gu.fold_norm(gt)
    assert e.value.status == qw.ERR_STATE
    q8 = qw.Weight.pack(ctx, D, qw.WFMT_INT8)
    with pytest.raises(qw.QwError) as e:
        q8.fold_norm(torch.zeros(I, device="cuda"))
    assert e.value.status == qw.ERR_DTYPE
    # an unfolded weight still needs gamma for the norm
    with pytest.raises(qw.QwError) as e:
        qw.linear(ctx, dn, torch.empty(1, I, device="cuda", dtype=torch.bfloat16),
                  torch.empty(1, H, device="cuda"), norm=True)
    assert e.value.status == qw.ERR_NULL


# ----------------------------------------------------------------------------
# stacked projections (qw_weight_pack_concat)
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("fmt", ["bf16", "int8"])
@pytest.mark.parametrize("M", [1, 40])
def test_pack_concat(qw, ctx, oracle, relerr, fmt, M):
    """in_proj_qkv + in_proj_z + in_proj_a + in_proj_b of a Gated-DeltaNet
    layer stacked into one weight: one launch, each part equal to its own
    projection (bitwise for the same kernel path) and to the FP64 reference."""
    K = 1024
    Ns = [6144, 2048, 16, 16]
    Ws = [oracle.normal((n, K), 900 + i, 0.0, 0.02) for i, n in enumerate(Ns)]
    f = qw.WFMT_BF16 if fmt == "bf16" else qw.WFMT_INT8
    xt = dev(oracle.normal((M, K), 910), torch.bfloat16 if fmt == "bf16" else torch.float16)
    cat = qw.Weight.pack_concat(ctx, Ws, f)
    y = torch.empty(M, sum(Ns), device="cuda")
    qw.linear(ctx, cat, xt, y)
    torch.cuda.synchronize()
    xs = host(xt)
    o = 0
    for i, (n, W) in enumerate(zip(Ns, Ws)):
        w1 = qw.Weight.pack(ctx, W, f)
        yi = torch.empty(M, n, device="cuda")
        qw.linear(ctx, w1, xt, yi)
        torch.cuda.synchronize()
        part = host(y)[:, o:o + n]
        if fmt == "bf16":
            ref = oracle.linear_f64(oracle.round_bf16(W), xs)
            assert relerr(part, ref) <= 2e-5
        else:
            ref = oracle.linear_int8_f64(*w1.unpack(), xs)
            assert relerr(part, ref) <= 1e-3
        o += n
    with pytest.raises(qw.QwError) as e:
        qw.Weight.pack_concat(ctx, [Ws[2][:10], Ws[3]], f)   # 10 rows: not a multiple of 16
    assert e.value.status == qw.ERR_SHAPE
