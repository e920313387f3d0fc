"""GPU parity of the direct-A GEMM's two block shapes (qw_gemm_da.hip): 4 waves
x 256 weight rows (two workgroups per CU) and 8 waves x 512 weight rows (one
per CU, the default where the 512-row blocks cover every CU).  Each output
element sums its k-steps in the same order in both shapes, so the two routes
must agree bit for bit; the 8-wave route is also checked against FP64 on the
stored BF16 operands.  QW_GEMM_DA=2 takes the direct-A route at every size,
QW_GEMM_DA_W8 forces the shape, QW_GEMM_DA_PERSIST the persistent form of
the 8-wave kernel (one workgroup per CU walking its XCD's blocks, the next
block's operands loaded during this block's epilogue).  Ragged shapes: partial 512-row blocks
(8224 and 1024 + 16 rows), partial token blocks, every epilogue (plain,
residual, GLU, Q/gate split).  Bars: <= 1e-5 normwise vs FP64 (FP32
outputs), 1e-4 for the GLU (SiLU of sums).
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


@pytest.fixture(scope="module")
def ctx_w(qw):
    """Contexts by forced block shape (4 or 8 waves, "p": 8 waves as the
    persistent kernel), direct-A at every size."""
    made = {}

    def get(nw):
        if nw not in made:
            keys = {"QW_GEMM_DA": "2", "QW_GEMM_DA_W8": "0" if nw == 4 else "1",
                    "QW_GEMM_DA_PERSIST": "1" if nw == "p" else "0"}
            old = {k: os.environ.get(k) for k in keys}
            os.environ.update(keys)
            try:
                made[nw] = qw.Context(0)
            finally:
                for k, v in old.items():
                    if v is None:
                        os.environ.pop(k, None)
                    else:
                        os.environ[k] = v
        return made[nw]
    yield get
    for c in made.values():
        c.close()


def _both(qw, ctx_w, pack, run):
    """run(ctx, weight) -> output tensors, for 8 waves (one launch per block
    and persistent) and 4 waves."""
    outs = {}
    for nw in (8, "p", 4):
        c = ctx_w(nw)
        outs[nw] = run(c, pack(c))
        torch.cuda.synchronize()
        assert c.device_error() == 0
    for a, b in zip(outs[8], outs[4]):
        assert torch.equal(a, b), "8-wave and 4-wave blocks differ"
    for a, b in zip(outs["p"], outs[4]):
        assert torch.equal(a, b), "persistent 8-wave and 4-wave blocks differ"
    return outs[8]


@pytest.mark.parametrize("N,M", [(8224, 1000), (1040, 520), (4096, 777)])
def test_waves_plain(qw, ctx_w, oracle, relerr, N, M):
    W = oracle.normal((N, 1024), 7300 + N, 0.0, 0.02)
    x = oracle.normal((M, 1024), 7301 + M)
    xt = dev(x, torch.bfloat16)

    def run(c, w):
        y = torch.empty(M, N, device="cuda")
        qw.linear(c, w, xt, y)
        return [y]
    (y,) = _both(qw, ctx_w, lambda c: qw.Weight.pack(c, W, qw.WFMT_BF16), run)
    assert relerr(host(y), oracle.linear_f64(oracle.round_bf16(W), host(xt))) <= 1e-5


@pytest.mark.parametrize("K,M", [(2048, 777), (3584, 1536)])
def test_waves_residual(qw, ctx_w, oracle, relerr, K, M):
    W = oracle.normal((1024, K), 7310 + K, 0.0, 0.02)
    x = oracle.normal((M, K), 7311 + M)
    r = oracle.normal((M, 1024), 7312)
    xt = dev(x, torch.bfloat16)

    def run(c, w):
        y = dev(r)
        qw.linear(c, w, xt, y, residual=y)
        return [y]
    (y,) = _both(qw, ctx_w, lambda c: qw.Weight.pack(c, W, qw.WFMT_BF16), run)
    ref = oracle.linear_f64(oracle.round_bf16(W), host(xt)) + r
    assert relerr(host(y), ref) <= 1e-5


def test_waves_glu(qw, ctx_w, oracle, relerr):
    I, H, M = 3584, 1024, 640
    G = oracle.normal((I, H), 7320, 0.0, 0.02)
    U = oracle.normal((I, H), 7321, 0.0, 0.02)
    xt = dev(oracle.normal((M, H), 7322), torch.bfloat16)

    def run(c, w):
        h = torch.empty(M, I, device="cuda")
        qw.linear(c, w, xt, h)
        return [h]
    (h,) = _both(qw, ctx_w, lambda c: qw.Weight.pack_glu(c, G, U, qw.WFMT_BF16), run)
    xs = host(xt).astype(np.float64)
    g = xs @ oracle.round_bf16(G).astype(np.float64).T
    u = xs @ oracle.round_bf16(U).astype(np.float64).T
    assert relerr(host(h), g / (1.0 + np.exp(-g)) * u) <= 1e-4


def test_waves_q_gate(qw, ctx_w, oracle, relerr):
    heads, D, K, M = 8, 256, 1024, 520
    W = oracle.normal((2 * heads * D, K), 7330, 0.0, 0.02)
    xt = dev(oracle.normal((M, K), 7331), torch.bfloat16)

    def run(c, w):
        q = torch.empty(M, heads * D, device="cuda")
        g = torch.empty(M, heads * D, device="cuda")
        qw.linear(c, w, xt, q, y2=g, split_period=D)
        return [q, g]
    q, g = _both(qw, ctx_w, lambda c: qw.Weight.pack(c, W, qw.WFMT_BF16), run)
    full = oracle.linear_f64(oracle.round_bf16(W), host(xt))
    q_ref, g_ref = oracle.split_q_gate(full.astype(np.float32), heads, D)
    assert relerr(host(q), q_ref) <= 1e-5 and relerr(host(g), g_ref) <= 1e-5


@pytest.mark.parametrize("N,K,M,pad", [(8224, 1024, 1000, 72), (5120, 1024, 1536, 72), (4096, 2048, 777, 72),
                                       (1040, 512, 900, 72), (4096, 1024, 1100, 4)])
def test_waves_bf16_rows(qw, ctx_w, oracle, relerr, N, K, M, pad):
    """BF16 outputs into a wider row stride (the prefill's stacked input
    projections write y[:, :N] of a [M][8192+] buffer): the persistent kernel
    keeps half of each block's outputs in LDS and stores them during the next
    block's k-steps (K >= 1024), so ragged token and row blocks, a K of 2048
    (stores spread over the first 32 of 64 k-steps) and K = 512 (stored at
    once) are covered, and a row stride that is not a multiple of 8 (rows
    not 16-byte aligned: stored at once); the bytes past N of every row stay
    untouched."""
    W = oracle.normal((N, K), 7340 + N + K, 0.0, 0.02)
    xt = dev(oracle.normal((M, K), 7341 + M), torch.bfloat16)
    ld = N + pad

    def run(c, w):
        big = torch.full((M, ld), 7.0, device="cuda", dtype=torch.bfloat16)
        qw.linear(c, w, xt, big[:, :N], ldy=ld)
        return [big]
    (big,) = _both(qw, ctx_w, lambda c: qw.Weight.pack(c, W, qw.WFMT_BF16), run)
    assert bool((big[:, N:] == 7.0).all()), "stores past N"
    assert relerr(host(big[:, :N]), oracle.linear_f64(oracle.round_bf16(W), host(xt))) <= 4e-3


@pytest.mark.parametrize("M", [640, 1300])
def test_waves_glu_bf16(qw, ctx_w, oracle, relerr, M):
    """GLU with BF16 outputs: the persistent kernel defers all of a block's
    256 x 128 outputs to the next block's k-steps."""
    I, H = 3584, 1024
    G = oracle.normal((I, H), 7350, 0.0, 0.02)
    U = oracle.normal((I, H), 7351, 0.0, 0.02)
    xt = dev(oracle.normal((M, H), 7352 + M), torch.bfloat16)

    def run(c, w):
        h = torch.empty(M, I, device="cuda", dtype=torch.bfloat16)
        qw.linear(c, w, xt, h)
        return [h]
    (h,) = _both(qw, ctx_w, lambda c: qw.Weight.pack_glu(c, G, U, qw.WFMT_BF16), run)
    xs = host(xt).astype(np.float64)
    g = xs @ oracle.round_bf16(G).astype(np.float64).T
    u = xs @ oracle.round_bf16(U).astype(np.float64).T
    assert relerr(host(h), g / (1.0 + np.exp(-g)) * u) <= 4e-3


@pytest.mark.parametrize("K,M", [(2048, 777), (3584, 1536), (2048, 4100)])
def test_waves_residual_bf16_inplace(qw, ctx_w, oracle, relerr, K, M):
    """BF16 residual added in place (y = residual), the prefill's out and
    down projections: the persistent kernel brings the residual rows of
    tokens 64..127 of each block into LDS before the block's k-loop."""
    W = oracle.normal((1024, K), 7360 + K, 0.0, 0.02)
    xt = dev(oracle.normal((M, K), 7361 + M), torch.bfloat16)
    r = dev(oracle.normal((M, 1024), 7362), torch.bfloat16)

    def run(c, w):
        y = r.clone()
        qw.linear(c, w, xt, y, residual=y)
        return [y]
    (y,) = _both(qw, ctx_w, lambda c: qw.Weight.pack(c, W, qw.WFMT_BF16), run)
    ref = oracle.linear_f64(oracle.round_bf16(W), host(xt)) + host(r)
    assert relerr(host(y), ref) <= 4e-3
