"""A kernel's first launch may happen inside a graph capture (qw_graph_begin):
the launchers that raise a kernel's dynamic-LDS limit on first use must not
invalidate the capture (that attribute call was once made in the capture's
thread-local mode, and the capture failed at qw_graph_end).

Kernels configure themselves once per process, so the check runs in a fresh
Python process: it captures the first-ever calls of the weight-stationary
projection (1024 x 2048, 17 tokens, residual), the direct-A GEMM (2048
tokens), the skinny kernel (8 tokens) and the persistent MLP stack, replays
the graph three times, and compares every replay with eager calls of the same
operations (bit-identical: same kernels, same inputs).
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r'''
import importlib.util, sys, torch
spec = importlib.util.spec_from_file_location("qw", sys.argv[1])
qw = importlib.util.module_from_spec(spec); spec.loader.exec_module(qw)
ctx = qw.Context(0)
g = torch.Generator(device="cuda").manual_seed(7)
r = lambda *s, std=1.0: (torch.randn(*s, generator=g, device="cuda") * std).to(torch.bfloat16)
H, I = 1024, 3584
w_out = qw.Weight.pack_device(ctx, r(1024, 2048, std=0.02), qw.WFMT_BF16)
w_in = qw.Weight.pack_device(ctx, r(8192, 1024, std=0.02), qw.WFMT_BF16)
gu = [qw.Weight.pack_glu_device(ctx, r(I, H, std=0.02), r(I, H, std=0.02), qw.WFMT_BF16) for _ in range(2)]
dn = [qw.Weight.pack_device(ctx, r(H, I, std=0.02), qw.WFMT_BF16) for _ in range(2)]
gam = [(torch.randn(H, generator=g, device="cuda") * 0.02).float() for _ in range(2)]
a17, res17 = r(17, 2048), r(17, 1024)
x2k = r(2048, 1024)
x8 = r(8, 1024)
h1 = r(1, 1024)
y17 = torch.empty(17, 1024, device="cuda", dtype=torch.bfloat16)
y2k = torch.empty(2048, 8192, device="cuda", dtype=torch.bfloat16)
y8 = torch.empty(8, 8192, device="cuda", dtype=torch.bfloat16)
hs = torch.empty(1, 1024, device="cuda", dtype=torch.bfloat16)
torch.cuda.synchronize()
s = torch.cuda.Stream()
def body():
    qw.linear(ctx, w_out, a17, y17, residual=res17, stream=s)
    qw.linear(ctx, w_in, x2k, y2k, stream=s)
    qw.linear(ctx, w_in, x8, y8, stream=s)
    qw.mlp_stack(ctx, gu, dn, h1, hs, gammas=gam, stream=s)
with torch.cuda.stream(s):
    gr = qw.Graph(ctx, s)
    with gr:
        body()
outs = (y17, y2k, y8, hs)
for rep in range(3):
    for t in outs: t.zero_()
    with torch.cuda.stream(s):
        gr.launch(s)
    s.synchronize()
    got = [t.clone() for t in outs]
    for t in outs: t.zero_()
    with torch.cuda.stream(s):
        body()
    s.synchronize()
    for a, b in zip(got, outs):
        assert torch.equal(a, b), "graph replay %d differs from the eager calls" % rep
        assert float(b.float().abs().sum()) > 0.0
assert ctx.device_error() == 0
print("first-use capture ok", flush=True)
'''


def test_first_launch_inside_capture():
    pkg = os.path.join(ROOT, "qwen3.5_0.8b_deploy_amd", "qw.py")
    p = subprocess.run([sys.executable, "-c", SCRIPT, pkg], capture_output=True, text=True, timeout=110)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-3000:]
    assert "first-use capture ok" in p.stdout
