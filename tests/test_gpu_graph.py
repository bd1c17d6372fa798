"""HIP graph capture: calls recorded once and replayed, each replay (with new
inputs and eager work in between) checked against an eager call on the same
inputs.

- tt_mp2_energy_noalloc allocates nothing and clears its accumulator with a
  kernel (no memset node); bitwise in deterministic mode.
- einsum on GEMM, batched, strided, permutation, fused-path and 16-bit
  contractions, and the public mp2_energy with and without its row-padded
  copy of B: outputs and workspaces come from torch's graph pool; bitwise.
"""

import pytest
import torch

from trntensor_amd.hip import _lib, engine

pytestmark = pytest.mark.gpu


def _inputs(seed, nocc=10, nvir=130, naux=96):
    g = torch.Generator().manual_seed(seed)
    B = torch.randn(nocc, nvir, naux, generator=g, dtype=torch.float64) * 0.05
    eo = torch.sort(-20 + 19.7 * torch.rand(nocc, generator=g, dtype=torch.float64))[0]
    ev = torch.sort(0.1 + 4.9 * torch.rand(nvir, generator=g, dtype=torch.float64))[0]
    return B.cuda(), eo.cuda(), ev.cuda()


def _eager(lib, B, eo, ev):
    nocc, nvir, naux = B.shape
    wsb = lib.tt_mp2_energy_workspace_bytes(_lib.TT_F64, nocc, nvir, naux)
    ws = torch.empty(int(wsb), dtype=torch.uint8, device="cuda")
    e = torch.empty((), dtype=torch.float64, device="cuda")
    st = lib.tt_mp2_energy(_lib.TT_F64, nocc, nvir, naux, B.data_ptr(), eo.data_ptr(), ev.data_ptr(), e.data_ptr(),
                           ws.data_ptr(), wsb, 1, engine._stream_ptr(B.device))
    _lib.check(st, "tt_mp2_energy")
    torch.cuda.synchronize()
    return float(e)


@pytest.mark.parametrize("deterministic", [1, 0])
def test_noalloc_graph_replays(hip, deterministic):
    lib = _lib.load()
    B, eo, ev = _inputs(0)
    nocc, nvir, naux = B.shape
    e = torch.full((), float("nan"), dtype=torch.float64, device="cuda")

    def call():
        st = lib.tt_mp2_energy_noalloc(_lib.TT_F64, nocc, nvir, naux, B.data_ptr(), eo.data_ptr(), ev.data_ptr(),
                                       e.data_ptr(), deterministic, engine._stream_ptr(B.device))
        _lib.check(st, "tt_mp2_energy_noalloc")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()  # warm-up outside capture: looks up the scratch address once
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for k in range(4):
        src = _inputs(k + 1)
        B.copy_(src[0])
        eo.copy_(src[1])
        ev.copy_(src[2])
        torch.cuda.synchronize()
        want = _eager(lib, B, eo, ev)  # eager work between replays
        print(f"graph replay {k} deterministic={deterministic}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        got = float(e)
        if deterministic:
            assert got == want, (k, got, want)
        else:
            assert abs(got - want) <= 1e-12 * abs(want), (k, got, want)


@pytest.mark.parametrize(
    "sub,shapes,kw",
    [
        ("ij,jk->ik", [(200, 150), (150, 170)], {"alpha": 1.5, "beta": 0.5, "out": (200, 170)}),
        ("bij,bjk->bik", [(4, 64, 80), (4, 80, 48)], {}),
        ("mi,mnP->inP", [(40, 8), (40, 40, 24)], {}),
        ("ijk->k", [(30, 40, 500)], {}),
        ("ijk->kji", [(70, 80, 90)], {}),
        ("ia,jb,abP,ijP->", [(6, 7), (5, 9), (7, 9, 11), (6, 5, 11)], {}),
        ("ij,jk->ik", [(64, 64), (64, 96)], {"dtype": "bf16"}),
    ],
)
def test_einsum_graph_replays(hip, sub, shapes, kw):
    """einsum recorded once under torch.cuda.graph (the library allocates
    nothing and issues no memsets; outputs and workspaces come from torch's
    graph pool) replays with new operand values, each replay equal to an
    eager call on the same operands."""
    import trntensor_amd as tt

    g = torch.Generator().manual_seed(len(sub))
    ops = [torch.randn(*s, generator=g, dtype=torch.float64).cuda() for s in shapes]
    kw = dict(kw)
    if "out" in kw:
        kw["out"] = torch.randn(*kw["out"], generator=g, dtype=torch.float64).cuda()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        tt.einsum(sub, *ops, **kw)  # warm-up: plans and launch recipes cached outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        res = tt.einsum(sub, *ops, **kw)
    for k in range(3):
        for op, s in zip(ops, shapes):
            op.copy_(torch.randn(*s, generator=g, dtype=torch.float64))
        torch.cuda.synchronize()
        want = tt.einsum(sub, *ops, **kw).clone()
        print(f"einsum graph {sub} replay {k}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(res, want), (sub, k, (res.double() - want.double()).abs().max().item())


@pytest.mark.parametrize("naux", [96, 37])
def test_mp2_energy_graph_replays(hip, naux):
    """The public mp2_energy recorded once under torch.cuda.graph: with naux
    37 the call stages B into its workspace with rows padded to 48 elements
    (a copy kernel, then the energy and the fixed-order sum), with naux 96 it
    runs on B as given. Each replay, with new inputs and eager work in
    between, equals an eager call bitwise."""
    import trntensor_amd as tt

    B, eo, ev = _inputs(0, naux=naux)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        tt.mp2_energy(B, eo, ev)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        res = tt.mp2_energy(B, eo, ev)
    for k in range(3):
        src = _inputs(k + 1, naux=naux)
        B.copy_(src[0])
        eo.copy_(src[1])
        ev.copy_(src[2])
        torch.cuda.synchronize()
        want = float(tt.mp2_energy(B, eo, ev))
        print(f"mp2_energy graph naux={naux} replay {k}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert float(res) == want, (naux, k, float(res), want)
