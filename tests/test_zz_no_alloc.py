"""GPU check of qw_lmhead_argmax_noalloc, the entry point that allocates
nothing (its argmax keys live in a fixed per-device array inside the
library), against qw_lmhead_argmax on the same packed weights: identical ids
and winning logits, bit for bit, on two calls in a row (the second with fewer
tokens, so stale keys of the first would show), over BF16 and INT8 weights
and both routes (M = 32, 128, 200: the weight-stationary argmax kernel;
M = 5: the small-M kernels).  Called through the C ABI (ctypes)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.mark.parametrize("fmt", ["bf16", "int8"])
def test_noalloc_matches_lmhead_argmax(qw, ctx, oracle, fmt):
    V, K = 40000, 1024
    E = oracle.normal((V, K), 1501, 0.0, 0.02)
    wf = qw.WFMT_BF16 if fmt == "bf16" else qw.WFMT_INT8
    w = qw.Weight.pack(ctx, E, wf)
    hdt = torch.bfloat16 if fmt == "bf16" else torch.float16
    for M, seed in ((200, 1505), (128, 1502), (5, 1503), (32, 1504)):
        h = torch.from_numpy(oracle.normal((M, K), seed)).cuda().to(hdt)
        ids_a = torch.full((M,), -1, dtype=torch.int32, device="cuda")
        mx_a = torch.empty(M, device="cuda")
        qw.lmhead_argmax(ctx, w, h, ids_a, mx_a)
        ids_b = torch.full((M,), -1, dtype=torch.int32, device="cuda")
        mx_b = torch.empty(M, device="cuda")
        qw.lmhead_argmax_noalloc(w, h, ids_b, mx_b)
        torch.cuda.synchronize()
        assert torch.equal(ids_a, ids_b), (M, fmt)
        assert torch.equal(mx_a, mx_b), (M, fmt)
        assert int(ids_b.min()) >= 0


def test_noalloc_rejects_beyond_max(qw, ctx, oracle):
    V, K = 1000, 128
    w = qw.Weight.pack(ctx, oracle.normal((V, K), 1510, 0.0, 0.02), qw.WFMT_BF16)
    h = torch.zeros(257, K, device="cuda", dtype=torch.bfloat16)
    ids = torch.empty(257, dtype=torch.int32, device="cuda")
    with pytest.raises(qw.QwError) as e:
        qw.lmhead_argmax_noalloc(w, h, ids)
    assert e.value.status == qw.ERR_SHAPE


@pytest.mark.parametrize("M", [1, 64, 100])
def test_noalloc_graph_replays(qw, ctx, oracle, M):
    """Captured once in a graph (the use the entry point exists for) and
    replayed with new activations copied in between, eager work of the
    program between the replays: every replay's ids and winning logits equal
    an eager qw_lmhead_argmax on the same activations."""
    V, K = 30000, 1024
    w = qw.Weight.pack(ctx, oracle.normal((V, K), 1520, 0.0, 0.02), qw.WFMT_BF16)
    h = torch.zeros(M, K, device="cuda", dtype=torch.bfloat16)
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    mx = torch.empty(M, device="cuda")
    stream = torch.cuda.Stream()
    g = qw.Graph(ctx, stream)
    with torch.cuda.stream(stream):
        stream.synchronize()
        with g:
            qw.lmhead_argmax_noalloc(w, h, ids, mx, stream=stream)
    for rep in range(4):
        hv = torch.from_numpy(oracle.normal((M, K), 1530 + rep)).cuda().to(torch.bfloat16)
        h.copy_(hv)
        torch.cuda.synchronize()
        g.launch(stream)
        stream.synchronize()
        ids_e = torch.full((M,), -1, dtype=torch.int32, device="cuda")
        mx_e = torch.empty(M, device="cuda")
        qw.lmhead_argmax(ctx, w, hv, ids_e, mx_e)
        torch.cuda.synchronize()
        assert torch.equal(ids, ids_e), rep
        assert torch.equal(mx, mx_e), rep
