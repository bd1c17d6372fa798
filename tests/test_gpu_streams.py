"""The library launches on torch's current stream: work issued inside
``torch.cuda.stream(s)`` is queued on s (s reports pending work right after
the call while the default stream is idle), ordered after s's earlier work,
and its results equal the same call on the default stream. Host threads on
their own streams get the same results as single-threaded calls."""

import pytest
import torch

import trntensor_amd as tt

pytestmark = pytest.mark.gpu


def _pending_on_side_stream(fn):
    """Run fn() under a side stream; return (side busy, default busy) right after."""
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        out = fn()
        side_busy = not side.query()
    default_busy = not torch.cuda.default_stream().query()
    side.synchronize()
    return out, side_busy, default_busy


def test_einsum_gemm_runs_on_the_current_stream(hip):
    g = torch.Generator(device="cuda").manual_seed(3)
    # 8192^3 fp64: about 17 ms of MFMA work, long enough to still be running
    # when the host queries the streams.
    A = torch.randn(8192, 8192, device="cuda", dtype=torch.float64, generator=g)
    B = torch.randn(8192, 8192, device="cuda", dtype=torch.float64, generator=g)
    ref = tt.einsum("ij,jk->ik", A, B)
    torch.cuda.synchronize()
    out, side_busy, default_busy = _pending_on_side_stream(lambda: tt.einsum("ij,jk->ik", A, B))
    print(f"side busy {side_busy}, default busy {default_busy}")
    assert side_busy and not default_busy
    assert torch.equal(out, ref)


def test_mp2_energy_runs_on_the_current_stream(hip):
    g = torch.Generator().manual_seed(4)
    B = (torch.randn(64, 320, 1200, generator=g, dtype=torch.float64) * 0.05).cuda()
    eo = torch.sort(-20 + 19.7 * torch.rand(64, generator=g, dtype=torch.float64))[0].cuda()
    ev = torch.sort(0.1 + 4.9 * torch.rand(320, generator=g, dtype=torch.float64))[0].cuda()
    ref = tt.mp2_energy(B, eo, ev)
    torch.cuda.synchronize()
    out, side_busy, default_busy = _pending_on_side_stream(lambda: tt.mp2_energy(B, eo, ev))
    print(f"side busy {side_busy}, default busy {default_busy}")
    assert side_busy and not default_busy
    assert torch.equal(out, ref)


def test_side_stream_work_is_ordered_after_its_producer(hip):
    """Operands written by an earlier kernel on the same side stream are read
    after it finishes (no synchronisation in between)."""
    g = torch.Generator(device="cuda").manual_seed(5)
    X = torch.randn(4096, 4096, device="cuda", dtype=torch.float64, generator=g)
    Y = torch.randn(4096, 4096, device="cuda", dtype=torch.float64, generator=g)
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        A = tt.einsum("ij,jk->ik", X, Y)  # producer, several ms
        A.mul_(0.5)  # torch kernel on the same stream
        C = tt.einsum("ij,jk->ik", A, Y)  # consumer
    side.synchronize()
    ref_a = tt.einsum("ij,jk->ik", X, Y) * 0.5
    ref = tt.einsum("ij,jk->ik", ref_a, Y)
    torch.cuda.synchronize()
    assert torch.equal(C, ref)


def test_threads_on_their_own_streams(hip):
    """Four host threads, each on its own stream (torch's current stream is
    per thread), run einsum and mp2_energy on their own inputs; every result
    equals the same call made alone on the main thread."""
    import threading

    def inputs(seed):
        g = torch.Generator().manual_seed(seed)
        A = torch.randn(512, 384, generator=g, dtype=torch.float64).cuda()
        Bm = torch.randn(384, 640, generator=g, dtype=torch.float64).cuda()
        Bov = (torch.randn(6, 100, 97, generator=g, dtype=torch.float64) * 0.05).cuda()
        eo = torch.sort(-20 + 19.7 * torch.rand(6, generator=g, dtype=torch.float64))[0].cuda()
        ev = torch.sort(0.1 + 4.9 * torch.rand(100, generator=g, dtype=torch.float64))[0].cuda()
        return A, Bm, Bov, eo, ev

    def work(A, Bm, Bov, eo, ev):
        return tt.einsum("ij,jk->ik", A, Bm), tt.mp2_energy(Bov, eo, ev)

    data = [inputs(100 + t) for t in range(4)]
    refs = [work(*d) for d in data]
    torch.cuda.synchronize()
    results = [[] for _ in data]
    errors = []

    def run(t):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(10):
                    results[t].append(work(*data[t]))
            s.synchronize()
        except Exception as exc:  # reported on the main thread
            errors.append(repr(exc))

    threads = [threading.Thread(target=run, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not errors, errors
    for t, (gemm_ref, e_ref) in enumerate(refs):
        assert len(results[t]) == 10
        for gemm, e in results[t]:
            assert torch.equal(gemm, gemm_ref)
            assert torch.equal(e, e_ref)
