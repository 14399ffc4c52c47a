"""rxq4_gemm_noalloc: the GEMM whose split partials live in the library's
fixed device array instead of an allocated workspace.  Called through the C
ABI and compared with rxq4_gemm (same routing and split plan, so the same
bits) and with the fp64 oracle at the GEMM bar, on two calls in a row with the
second one smaller; no device memory is allocated by it, also on a stream
that has never run a split launch, and it replays from a HIP graph.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rxq4 import capi
from tests import util

pytestmark = pytest.mark.gpu


def _weights(seed, M, K):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return capi.quantize(torch.randn((M, K), generator=g, device="cuda") * 0.02)


def _check_oracle(y32, W, x, M, K, seed):
    rows = np.sort(util.rng(seed).choice(M, 64, replace=False))
    Wn = W[torch.from_numpy(rows).cuda()].cpu().numpy()
    xv = x.float().cpu().numpy()
    kind = "bf16" if x.dtype == torch.bfloat16 else "f16"
    ref = orc.gemm_f64(Wn, K, xv, kind)
    assert util.rel_err(y32.cpu().numpy()[:, rows], ref) <= util.TOL


def test_gemm_noalloc_matches_gemm_two_calls_second_smaller():
    # call 1: [2048 x 11008] at m = 512 (split-K: 32 tiles x 8 splits, 32 MiB
    # of partials); call 2: [2048 x 11008] at m = 16 (K split over
    # workgroups, 0.5 MiB) -- it reads none of call 1's leftover partials
    cases = [(2048, 512, 11008, torch.bfloat16), (2048, 16, 11008, torch.float16)]
    s = torch.cuda.Stream()  # never used by a split launch: no workspace exists for it
    # the HIP runtime materialises the library's fixed array (48 MiB) when its
    # code object is first used on the device: do that before measuring
    Wt = _weights(899, 256, 256)
    xt = torch.zeros((32, 256), dtype=torch.bfloat16, device="cuda")
    capi.gemm_noalloc(torch.empty((32, 256), dtype=torch.bfloat16, device="cuda"), Wt, xt,
                      256, 32, 256)
    for i, (M, N, K, dt) in enumerate(cases):
        print(f"noalloc call {i}: M={M} N={N} K={K} {dt}", flush=True)
        W = _weights(900 + i, M, K)
        g = torch.Generator(device="cuda").manual_seed(910 + i)
        x = torch.randn((N, K), generator=g, device="cuda").to(dt)
        ref = torch.empty((N, M), dtype=dt, device="cuda")
        ref32 = torch.empty((N, M), dtype=torch.float32, device="cuda")
        capi.gemm(ref, W, x, M, N, K)
        capi.gemm(ref32, W, x, M, N, K)
        y = torch.full((N, M), 7.0, dtype=dt, device="cuda")
        y32 = torch.full((N, M), 7.0, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        with torch.cuda.stream(s):
            capi.gemm_noalloc(y, W, x, M, N, K, stream=s)
            capi.gemm_noalloc(y32, W, x, M, N, K, stream=s)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        # a workspace allocation for s would take 48 MiB
        assert free1 >= free0 - (4 << 20), (free0, free1)
        assert torch.equal(y, ref)
        assert torch.equal(y32, ref32)
        _check_oracle(y32, W, x, M, K, 920 + i)


def test_gemm_noalloc_replays_in_a_graph():
    M, N, K = 2048, 512, 11008
    W = _weights(930, M, K)
    g = torch.Generator(device="cuda").manual_seed(931)
    x = torch.randn((N, K), generator=g, device="cuda").to(torch.bfloat16)
    ref = torch.empty((N, M), dtype=torch.bfloat16, device="cuda")
    capi.gemm(ref, W, x, M, N, K)
    y = torch.empty_like(ref)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        capi.gemm_noalloc(y, W, x, M, N, K, stream=s)
    for rep in range(3):
        with torch.cuda.stream(s):
            y.fill_(0)
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), rep
        # eager use of the same array between replays
        y2 = torch.empty_like(ref)
        capi.gemm_noalloc(y2, W, x, M, N, K)
        torch.cuda.synchronize()
        assert torch.equal(y2, ref), rep


_FIRST_CALL_IN_CAPTURE = r"""
import sys
sys.path[:0] = sys.argv[1:3]
import torch
import rxq4
from rxq4 import capi
rxq4.load()
M, N, K = 2048, 512, 11008
g = torch.Generator(device="cuda").manual_seed(940)
W = capi.quantize(torch.randn((M, K), generator=g, device="cuda") * 0.02)
x = torch.randn((N, K), generator=g, device="cuda").to(torch.bfloat16)
ref = torch.empty((N, M), dtype=torch.bfloat16, device="cuda")
capi.gemm(ref, W, x, M, N, K)
y = torch.empty_like(ref)
torch.cuda.synchronize()
s = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
# the process's first rxq4_gemm_noalloc call: made while s is captured
# (torch's global capture mode)
with torch.cuda.graph(graph, stream=s):
    capi.gemm_noalloc(y, W, x, M, N, K, stream=s)
for rep in range(3):
    with torch.cuda.stream(s):
        y.fill_(0)
        graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, ref), rep
print("first-call-in-capture ok", flush=True)
"""


def test_gemm_noalloc_first_call_inside_a_capture():
    """A fresh process whose first rxq4_gemm_noalloc call happens inside a
    torch graph capture (the lookup of the array's device address runs then):
    the graph replays bit for bit what rxq4_gemm computes."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    p = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, root,
                        os.path.join(root, "reflex-infer_amd")],
                       capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-4000:]
    assert "first-call-in-capture ok" in p.stdout
