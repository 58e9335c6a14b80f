"""zest_gemm_group_noalloc (the GEMM for callers that cannot allocate)
against zest_gemm_group: the same plan, so the same bits, on two calls in a
row (the second smaller, so the static workspace holds the first call's
partial sums when it starts), both within the GEMM bar of the oracle; no
device memory is allocated by the calls; a plan that needs more workspace than
the static array holds is refused before anything runs; captured in a HIP
graph, every replay gives the same bits."""
from __future__ import annotations

import numpy as np
import pytest
from gen import Rng, wide_blocks
from helpers import gemm_check

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _case(z, M, ns, K, seed):
    x = Rng(seed).normal(M * K).reshape(M, K)
    a = z.pack_act_x(_dev(x))
    ws = []
    for i, n in enumerate(ns):
        w = Rng(seed + 1 + i).normal(n * K, 0, 0.02).reshape(n, K)
        ws.append(z.convert_weight(0, _dev(w.view(np.uint8)), n, K))
    return a, ws


def test_noalloc_matches_gemm_group(zest_gpu, oracle):
    import torch
    z = zest_gpu
    # a down projection's shape whose weight is not whole 160-row tiles (152
    # tiles of 256 x 128: its plan splits K three ways, 57 MiB of partial
    # sums), then a smaller split-K group of two weights
    cases = [(2048, [2432], 9728, 5), (600, [1000, 520], 8192, 9)]
    prepared = [(M, ns, K, *_case(z, M, ns, K, seed)) for M, ns, K, seed in cases]
    wants = []
    for M, ns, K, a, ws in prepared:
        wants.append([o.clone() for o in z.gemm_group(a, M, ws, ns, K)])
    # every tensor the calls use exists before the free memory is read
    outs = [[torch.full((M, n), float("nan"), device="cuda") for n in ns] for M, ns, K, _, _ in prepared]
    flags = [torch.zeros(1, dtype=torch.int32, device="cuda") for _ in prepared]
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for (M, ns, K, a, ws), o, nf in zip(prepared, outs, flags):
        z.gemm_group(a, M, ws, ns, K, outs=o, nonfinite=nf, noalloc=True)
        torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0, "the no-alloc calls changed the free device memory"
    assert all(int(nf.item()) == 0 for nf in flags)
    for (M, ns, K, a, ws), want, got in zip(prepared, wants, outs):
        rows = np.unique(np.linspace(0, M - 1, 24).astype(int))
        ad = z.expanded_to_rows(a.cpu().numpy(), M, K)[rows]
        for i, n in enumerate(ns):
            assert torch.equal(got[i].view(torch.int32), want[i].view(torch.int32)), (M, n, K)
            wd = oracle.decode_rows(z.tiles_to_blocks(ws[i].cpu().numpy(), n, K))
            r64, ab = oracle.mul_mat_f64(wd, ad)
            worst, maxrel = gemm_check(got[i].cpu().numpy()[rows], r64, ab, K)
            assert worst <= 1.0 and maxrel <= 1e-3, (M, n, K, worst, maxrel)


def test_noalloc_refuses_a_plan_beyond_its_workspace(zest_gpu):
    # 2048 x 2816 over K = 65536: 176 whole tiles of 1024 K-steps for 256
    # CUs, which the planner splits several ways (at four or more, over 88 MiB
    # of partial sums, more than the 64 MiB array); zest_gemm_group allocates
    # that, the no-alloc entry point refuses before launching anything
    import torch
    z = zest_gpu
    M, N, K = 2048, 2816, 65536
    a = z.empty_act(M, K)
    a.zero_()
    w = z.empty_packed(N, K)
    w.zero_()
    out = torch.full((M, N), 7.0, device="cuda")
    with pytest.raises(RuntimeError, match="static workspace"):
        z.gemm_group(a, M, [w], [N], K, outs=[out], noalloc=True)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
    # the allocating entry point runs the same plan
    c = z.gemm_group(a, M, [w], [N], K)[0]
    torch.cuda.synchronize()
    assert bool((c == 0).all())


def test_noalloc_random_shapes(zest_gpu):
    # seeded shapes across the planner's tile shapes, K splits and K-groups,
    # on operands where a change of summation order shows: the no-alloc entry
    # point gives zest_gemm_group's bits (or refuses a plan beyond its array)
    import torch
    z = zest_gpu
    rng = np.random.default_rng(4242)
    for case in range(16):
        M = int(rng.choice([1, 65, 256, 600, 1024, 2048, 4096]))
        N = int(rng.integers(1, 96)) * 32
        K = int(rng.integers(1, 64)) * 64
        a = z.pack_act_x(_dev(wide_blocks(M, K, 500 + case)))
        w = z.convert_weight(0, _dev(wide_blocks(N, K, 600 + case, 0.05).view(np.uint8)), N, K)
        want = z.gemm_group(a, M, [w], [N], K)[0]
        try:
            got = z.gemm_group(a, M, [w], [N], K, noalloc=True)[0]
        except RuntimeError as e:
            assert "static workspace" in str(e), (M, N, K, str(e))
            continue
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (M, N, K)


def test_noalloc_under_graph_capture(zest_gpu):
    # the callers it is for: the no-alloc GEMM captured in a HIP graph (a
    # split-K plan, so the graph holds the kernel that clears the static
    # counters, not a memset), replayed three times with eager work between
    # the replays (the output poisoned); every replay gives the eager
    # allocating call's bits
    import torch
    z = zest_gpu
    M, ns, K = 2048, [2432], 9728
    a, ws = _case(z, M, ns, K, 5)
    want = z.gemm_group(a, M, ws, ns, K)[0].clone()
    out = torch.empty((M, ns[0]), device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        z.gemm_group(a, M, ws, ns, K, outs=[out], noalloc=True)   # the device's array looked up before capture
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        z.gemm_group(a, M, ws, ns, K, outs=[out], noalloc=True)
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), rep
        # eager work on the same array between replays
        z.gemm_group(a, 600, ws, ns, K, outs=[torch.empty((600, ns[0]), device="cuda")], noalloc=True)
        torch.cuda.synchronize()
