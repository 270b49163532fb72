"""mamw_muon_step_noalloc (workspace in the library's static device scratch)
against mamw_muon_step (caller workspace) through the C ABI: three calls in a
row on one GPU, each smaller than the one before (the last with ragged,
padded tiles on top of what the larger calls left in the scratch), each
bit-identical to the existing entry point in parameters, momentum and the
update buffer (same kernels, same launch plan); and one call captured in a
HIP graph and replayed with new gradients, each replay bit-identical to an
eager mamw_muon_step on the same values."""

import ctypes

import pytest
import torch

from triton_muon_adamw import _lib

pytestmark = pytest.mark.gpu

COEFFS = (3.4445, -4.7750, 2.0315)


def _twins(shapes, dev, seed):
    gen = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for shape in shapes:
        p = torch.empty(shape, device=dev).normal_(0.0, 0.02, generator=gen)
        g = torch.empty(shape, device=dev).normal_(0.0, 1.0, generator=gen)
        m = torch.empty(shape, device=dev).normal_(0.0, 1e-3, generator=gen)
        out.append(([p.clone(), g.clone(), m.clone(), torch.zeros_like(p)],
                    [p.clone(), g.clone(), m.clone(), torch.zeros_like(p)]))
    return out


def _arr(sets):
    arr = (_lib.MuonMatrix * len(sets))()
    for i, (p, g, m, u) in enumerate(sets):
        r, c = p.shape
        arr[i] = _lib.MuonMatrix(p.data_ptr(), g.data_ptr(), m.data_ptr(), u.data_ptr(), r, c,
                                 1e-2 * max(1.0, r / c) ** 0.5, 0)
    return arr


@pytest.mark.parametrize("calls", [[[(768, 3072), (3072, 768), (768, 3072)], [(256, 512), (512, 256)],
                                    [(200, 333), (333, 200)]]])
def test_noalloc_equals_workspace_step(gpu, calls):
    lib = _lib.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    for k, shapes in enumerate(calls):
        pairs = _twins(shapes, gpu, seed=40 + k)
        mine, ref = [a for a, _ in pairs], [b for _, b in pairs]
        n = len(shapes)
        nbytes = ctypes.c_size_t()
        _lib.check(lib.mamw_muon_workspace_bytes(n, shapes[0][0], shapes[0][1], 5, ctypes.byref(nbytes)), "ws")
        ws = torch.empty(nbytes.value, dtype=torch.uint8, device=gpu)
        st = lib.mamw_muon_step(_arr(ref), n, 1e-2, 0.1, 0.95, 1, *COEFFS, 5, 1e-7, ws.data_ptr(), nbytes.value,
                                stream)
        _lib.check(st, "mamw_muon_step")
        st = lib.mamw_muon_step_noalloc(_arr(mine), n, 1e-2, 0.1, 0.95, 1, *COEFFS, 5, 1e-7, stream)
        _lib.check(st, "mamw_muon_step_noalloc")
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(mine, ref)):
            for idx, what in ((0, "param"), (2, "momentum"), (3, "update")):
                assert torch.equal(a[idx], b[idx]), (k, i, what)
            assert a[3].abs().sum() > 0, (k, i)  # the update was written


def test_noalloc_graph_replay_equals_eager_steps(gpu):
    """A mamw_muon_step_noalloc call captured in a HIP graph (after one eager
    call, which resolves the scratch address on this device), replayed three
    times with new gradients copied into the captured gradient buffers: after
    each replay, parameters, momentum and update equal those of eager
    mamw_muon_step calls on the same values, bit for bit."""
    lib = _lib.load()
    shapes = [(640, 384), (384, 640)]
    pairs = _twins(shapes, gpu, seed=50)
    mine, ref = [a for a, _ in pairs], [b for _, b in pairs]
    n = len(shapes)
    nbytes = ctypes.c_size_t()
    _lib.check(lib.mamw_muon_workspace_bytes(n, 640, 384, 5, ctypes.byref(nbytes)), "ws")
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=gpu)
    arr_mine, arr_ref = _arr(mine), _arr(ref)

    def eager_ref():
        st = lib.mamw_muon_step(arr_ref, n, 1e-2, 0.1, 0.95, 1, *COEFFS, 5, 1e-7, ws.data_ptr(), nbytes.value,
                                torch.cuda.current_stream(gpu).cuda_stream)
        _lib.check(st, "mamw_muon_step")

    def noalloc_mine():
        st = lib.mamw_muon_step_noalloc(arr_mine, n, 1e-2, 0.1, 0.95, 1, *COEFFS, 5, 1e-7,
                                        torch.cuda.current_stream(gpu).cuda_stream)
        _lib.check(st, "mamw_muon_step_noalloc")

    eager_ref()
    noalloc_mine()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        noalloc_mine()
    gen = torch.Generator(device=gpu).manual_seed(51)
    for rep in range(3):
        for a, b in zip(mine, ref):
            g = torch.empty(a[1].shape, device=gpu).normal_(0.0, 1.0, generator=gen)
            a[1].copy_(g)
            b[1].copy_(g)
        torch.cuda.synchronize()
        graph.replay()
        eager_ref()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(mine, ref)):
            for idx, what in ((0, "param"), (2, "momentum"), (3, "update")):
                assert torch.equal(a[idx], b[idx]), (rep, i, what)
