"""Muon branch on the gfx950 kernels.

Drop-in for the reference's ``TritonMuon`` (muon/triton_muon.py:375-456) and its
launchers ``solve_ns_kernel_{1,2,3}`` (:95-117, :191-212, :281-310),
``newton_shultz_step`` (:313-325) and ``muon_step`` (:327-372).

``HipMuon.step()`` groups the matrices that have a gradient by
``(min(R,C), max(R,C))`` and runs each group as batched launches of
``mamw_muon_step`` (at most 32 matrices and a bounded workspace per call):
prep (momentum, Nesterov, bf16, transpose, sum of squares), norm, scale
(``X / ||X||`` in bf16 and its transpose), then per Newton-Schulz iteration a
Gram, a polynomial and an update GEMM, the last of which writes the
parameters.  The reference runs about 30 launches per matrix; here a group of
up to 32 matrices costs ``3 + 3*ns_steps`` launches.
Small steps (``HipMuon.concurrent_flops_limit``) run the shape groups
concurrently on side streams forked from and joined back into the caller's
current stream; the results are the same bits as in order.

Semantics kept from the reference: the constructor signature and defaults,
``AssertionError`` for an unknown ``adjust_lr_fn`` (:392-393) and for a
non-2-D parameter at step time (:96-97), momentum buffers shaped like the
parameter (:407-412), ``grad is None`` skipped (:420-421), zero-filling
``zero_grad`` (:450-456), and weight decay with the unscaled ``lr`` (:370).
The numerics follow torch.optim.Muon (the reference's own correctness oracle):
see ``include/muonadamw_amd.h``.  Differences from the reference, each
matching torch: ``match_rms_adamw`` scales by ``0.2*sqrt(max(R,C))`` (the
reference raises ``TypeError``, :428) and ``ns_steps=0`` applies the
normalised momentum (the reference still runs one iteration, :360).
"""

from __future__ import annotations

import ctypes
import math
import os
from collections.abc import Iterable
from typing import Literal

import torch
import torch.nn as nn

from .. import _lib

_ADJUST_FNS = ["original", "match_rms_adamw", "spectral_unclamped"]


def scaled_lr(lr: float, adjust_lr_fn: str, rows: int, cols: int) -> float:
    """Shape-dependent Muon learning rate (triton_muon.py:424-431; torch/optim/_muon.py:73-84)."""
    if adjust_lr_fn == "original":
        return lr * math.sqrt(max(1, rows / cols))
    if adjust_lr_fn == "match_rms_adamw":
        return lr * (0.2 * math.sqrt(max(rows, cols)))
    return lr * math.sqrt(rows / cols)


def _check_matrix(t: torch.Tensor, name: str, dtype=torch.float32, bf16_ok: bool = False) -> None:
    _lib.require_gpu_tensor(t, name)
    if t.dtype != dtype and not (bf16_ok and t.dtype == torch.bfloat16):
        raise TypeError(f"{name} must be {dtype}{' or torch.bfloat16' if bf16_ok else ''} (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _workspace_bytes(batch: int, rows: int, cols: int, ns_steps: int) -> int:
    n = ctypes.c_size_t()
    _lib.check(_lib.load().mamw_muon_workspace_bytes(batch, rows, cols, ns_steps, ctypes.byref(n)),
               "mamw_muon_workspace_bytes")
    return n.value


# ---------------------------------------------------------------------------
# Standalone launchers (bf16 matrices).  The kernels need dimensions padded to
# multiples of 128 (reduction length: 64); inputs that are not are copied into
# zero-padded buffers, which leaves every product unchanged.

def _padded(x: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    if x.shape == (rows, cols) and x.is_contiguous():
        return x
    out = torch.zeros((rows, cols), dtype=x.dtype, device=x.device)
    out[: x.shape[0], : x.shape[1]] = x
    return out


def _rup(x: int, to: int) -> int:
    return (x + to - 1) // to * to


def _check_bf16_2d(x: torch.Tensor, name: str) -> None:
    if x.ndim != 2:
        raise AssertionError("Muon only supports 2D tensors")
    _lib.require_gpu_tensor(x, name)
    if x.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16 (got {x.dtype})")


def solve_ns_kernel_1(matrix: torch.Tensor, out: torch.Tensor) -> None:
    """out = matrix @ matrix.T for a bf16 m x k matrix (triton_muon.py:95-117)."""
    _check_bf16_2d(matrix, "matrix")
    m, k = matrix.shape
    mp, kp = _rup(m, 128), _rup(k, 64)
    X = _padded(matrix, mp, kp)
    A = torch.empty((mp, mp), dtype=torch.bfloat16, device=matrix.device)
    lib = _lib.load()
    with torch.cuda.device(matrix.device):
        st = lib.mamw_ns_gram(X.data_ptr(), A.data_ptr(), 1, mp, kp, _lib.stream_handle(matrix.device))
    _lib.check(st, "mamw_ns_gram")
    out.copy_(A[:m, :m])


def solve_ns_kernel_2(matrix: torch.Tensor, b: float, c: float, out: torch.Tensor) -> None:
    """out = b*A + c*(A @ A.T) for a symmetric bf16 m x m matrix A (triton_muon.py:191-212)."""
    _check_bf16_2d(matrix, "matrix")
    m = matrix.shape[0]
    mp = _rup(m, 128)
    A = _padded(matrix, mp, mp)
    B = torch.empty((mp, mp), dtype=torch.bfloat16, device=matrix.device)
    lib = _lib.load()
    with torch.cuda.device(matrix.device):
        st = lib.mamw_ns_poly(A.data_ptr(), B.data_ptr(), 1, mp, b, c, _lib.stream_handle(matrix.device))
    _lib.check(st, "mamw_ns_poly")
    out.copy_(B[:m, :m])


def _transpose(x: torch.Tensor) -> torch.Tensor:
    r, c = x.shape
    t = torch.empty((c, r), dtype=x.dtype, device=x.device)
    with torch.cuda.device(x.device):
        st = _lib.load().mamw_transpose_bf16(x.data_ptr(), t.data_ptr(), 1, r, c,
                                             _lib.stream_handle(x.device))
    _lib.check(st, "mamw_transpose_bf16")
    return t


def solve_ns_kernel_3(X: torch.Tensor, out_2: torch.Tensor, a: float, out: torch.Tensor) -> None:
    """out = a*X + out_2 @ X for bf16 X (m x n) and symmetric out_2 (m x m) (triton_muon.py:281-310)."""
    _check_bf16_2d(X, "X")
    _check_bf16_2d(out_2, "out_2")
    m, n = X.shape
    mp, np_ = _rup(m, 128), _rup(n, 128)
    Xp = _padded(X, mp, np_)
    Bp = _padded(out_2, mp, mp)
    XT = _transpose(Xp)
    O = torch.empty((mp, np_), dtype=torch.bfloat16, device=X.device)
    lib = _lib.load()
    with torch.cuda.device(X.device):
        st = lib.mamw_ns_update(Bp.data_ptr(), Xp.data_ptr(), XT.data_ptr(), O.data_ptr(), None, 1, mp, np_,
                                a, _lib.stream_handle(X.device))
    _lib.check(st, "mamw_ns_update")
    out.copy_(O[:m, :n])


def newton_shultz_step(X: torch.Tensor, a: float, b: float, c: float, out: torch.Tensor) -> None:
    """One Newton-Schulz iteration out = a*X + (b*A + c*A@A) @ X, A = X @ X.T (triton_muon.py:313-325)."""
    _check_bf16_2d(X, "X")
    m, n = X.shape
    mp, np_ = _rup(m, 128), _rup(n, 128)
    dev = X.device
    Xp = _padded(X, mp, np_)
    XT = _transpose(Xp)
    A = torch.empty((mp, mp), dtype=torch.bfloat16, device=dev)
    B = torch.empty((mp, mp), dtype=torch.bfloat16, device=dev)
    O = torch.empty((mp, np_), dtype=torch.bfloat16, device=dev)
    lib = _lib.load()
    with torch.cuda.device(dev):
        s = _lib.stream_handle(dev)
        _lib.check(lib.mamw_ns_gram(Xp.data_ptr(), A.data_ptr(), 1, mp, np_, s), "mamw_ns_gram")
        _lib.check(lib.mamw_ns_poly(A.data_ptr(), B.data_ptr(), 1, mp, b, c, s), "mamw_ns_poly")
        _lib.check(lib.mamw_ns_update(B.data_ptr(), Xp.data_ptr(), XT.data_ptr(), O.data_ptr(), None, 1, mp,
                                      np_, a, s), "mamw_ns_update")
    out.copy_(O[:m, :n])


def muon_step(weights: torch.Tensor, grad: torch.Tensor, momentum: torch.Tensor, beta: float, a: float,
              b: float, c: float, lr: float, scaled_lr: float, weight_decay: float, steps: int, eps: float,
              nesterov: bool, out: torch.Tensor | None = None) -> None:
    """One Muon update of one matrix in place (triton_muon.py:327-372).

    ``out`` (optional, fp32, shaped like ``weights``) receives the
    orthogonalised update, as the reference's ``out`` buffer does (:368).
    """
    if weights.ndim != 2:
        raise AssertionError("Muon only supports 2D tensors")
    for t, name in ((weights, "weights"), (grad, "grad"), (momentum, "momentum")):
        _check_matrix(t, name)
        if t.shape != weights.shape or t.device != weights.device:
            raise ValueError(f"{name} must match the weights' shape and device")
    if out is not None:
        _check_matrix(out, "out")
        if out.shape != weights.shape or out.device != weights.device:
            raise ValueError("out must match the weights' shape and device")
    R, C = weights.shape
    nbytes = _workspace_bytes(1, R, C, steps)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=weights.device)
    arr = (_lib.MuonMatrix * 1)()
    arr[0] = _lib.MuonMatrix(weights.data_ptr(), grad.data_ptr(), momentum.data_ptr(),
                             out.data_ptr() if out is not None else None, R, C, scaled_lr, 0)
    lib = _lib.load()
    with torch.cuda.device(weights.device):
        st = lib.mamw_muon_step(arr, 1, lr, weight_decay, beta, int(bool(nesterov)), a, b, c, steps, eps,
                                ws.data_ptr(), nbytes, _lib.stream_handle(weights.device))
    _lib.check(st, "mamw_muon_step")


def gemm_tile(m: int, n: int, batch: int) -> int:
    """The library's GEMM tile edge for a launch group (``mamw_plan.cpp``
    ``choose_tile``): 256 from m = 2048; from m = 1024 for batches of 8 or
    more when the 256 padding adds at most 1/16 to the 128 padding; else 128."""
    if m >= 2048:
        return 256
    rup = lambda x, t: -(-x // t) * t  # noqa: E731
    if m >= 1024 and batch >= 8 and rup(m, 256) * rup(n, 256) * 16 <= rup(m, 128) * rup(n, 128) * 17:
        return 256
    return 128


def group_sizes(count: int, cap: int, m: int, n: int, cus: int) -> list[int]:
    """Sizes of the launch groups for ``count`` matrices of one shape class
    (``m = min(R, C)``, ``n = max(R, C)``), each at most ``cap``.

    Every group runs its Gram, polynomial and update GEMMs as one grid each,
    and a grid whose workgroups do not fill whole rounds of the GPU's CU slots
    leaves CUs idle in its last round.  The cost of a group of k matrices is
    modelled as each product's rounds times its reduction length (Gram: n,
    polynomial and update: m) times the relative time of one k step of its
    tile (a 256 x 256 step, one workgroup per CU, counts 1.4 steps of the
    128 x 128 tile, two workgroups per CU), plus a quarter round of each
    product per group for its launches.  The cheapest split into groups of any
    sizes wins (ties: fewer groups), found by dynamic programming over the
    number of matrices covered.  Tiles follow the library's choice for the
    group's size (``gemm_tile``), and a group on the 128 tile takes 256 x 256
    updates from m = 1024 when both padded edges are multiples of 256.
    """
    if count <= 0:
        return []
    cap = max(1, min(cap, count))
    step = {128: 1.0, 256: 1.4}

    def cost(k: int) -> float:
        tile = gemm_tile(m, n, k)
        mp, np_ = -(-m // tile) * tile, -(-n // tile) * tile
        utile = 256 if (tile == 128 and m >= 1024 and mp % 256 == 0 and np_ % 256 == 0) else tile
        tm = mp // tile
        sym, upd = tm * (tm + 1) // 2, (mp // utile) * (np_ // utile)
        rounds = lambda tiles, t: -(-tiles * k // (cus * (1 if t == 256 else 2)))  # noqa: E731
        return (rounds(sym, tile) * step[tile] * (n + m) + rounds(upd, utile) * step[utile] * m
                + 0.25 * (step[tile] * (n + m) + step[utile] * m))

    # best[c]: (cost, number of groups, sizes) of the cheapest split of c matrices
    best: list = [(0.0, 0, [])] + [None] * count
    for c in range(1, count + 1):
        for k in range(1, min(cap, c) + 1):
            pc, pg, ps = best[c - k]
            cand = (pc + cost(k), pg + 1, ps + [k])
            cur = best[c]
            if cur is None or cand[0] < cur[0] - 1e-9 or (abs(cand[0] - cur[0]) <= 1e-9 and cand[1] < cur[1]):
                best[c] = cand
    return sorted(best[count][2], reverse=True)


def _launch_rounds(tiles: int, tile: int, k: int, cus: int) -> float:
    """Time of one GEMM launch in k steps of a 256-wide tile: whole rounds of
    the grid (two 128-wide workgroups per CU, a quarter of the work each)."""
    slots = cus * (2 if tile == 128 else 1)
    return math.ceil(tiles / slots) * (k / 64) * (1.0 if tile == 256 else 0.5)


def _class_time(calls, key, steps: int, cus: int) -> float:
    """Estimated Newton-Schulz time of one shape class (its launch groups one
    after another): a launch whose grid fills a fraction of the GPU still
    takes a round, which is what makes a class of small grids slow for its
    flops."""
    t = 0.0
    for c in calls:
        if (c.device, c.group) != key:
            continue
        tile = gemm_tile(c.m, c.n_, c.n)
        mp, np_ = -(-c.m // tile) * tile, -(-c.n_ // tile) * tile
        tm = mp // tile
        sym = c.n * tm * (tm + 1) // 2  # Gram and polynomial tiles (lower triangle)
        utile = 256 if (tile == 128 and c.m >= 1024 and mp % 256 == 0 and np_ % 256 == 0) else tile
        upd = c.n * (mp // utile) * (np_ // utile)
        t += steps * (_launch_rounds(sym, tile, np_, cus) + _launch_rounds(sym, tile, mp, cus)
                      + _launch_rounds(upd, utile, mp, cus))
    return t


def _lanes(calls, steps: int, cus: dict) -> tuple[dict, dict]:
    """Streams of concurrent shape classes, per device, and each class's
    estimated time (_class_time).  The longest class runs on the caller's
    stream (None); the others, longest first, each on the least loaded of
    L - 1 side streams of the library's own (_lib.side_streams), where a side
    stream's classes run one after another.  L is the fewest lanes (2 to 4)
    whose side streams all finish within the caller's class; more concurrent
    streams than that only contend.  Measured: config 3 (the 4096 x 14336
    class against four smaller ones) 4.91 ms with two lanes against 5.01 with
    one side stream per class; GPT-2 1.80 against 1.81; the reference's hybrid
    MLP (four batch-1 classes whose grids mostly underfill the GPU) needs
    three."""
    lanes: dict = {}
    times: dict = {}
    for dev in dict.fromkeys(c.device for c in calls):
        keys = list(dict.fromkeys((c.device, c.group) for c in calls if c.device == dev))
        for k in keys:
            times[k] = _class_time(calls, k, steps, cus[dev])
        keys.sort(key=lambda k: times[k], reverse=True)
        lanes[keys[0]] = None
        rest = keys[1:]
        if not rest:
            continue
        n_side, pick = _lane_split([times[k] for k in keys])
        streams = _lib.side_streams(dev, n_side)
        for k, i in zip(rest, pick):
            lanes[k] = streams[i]
    return lanes, times


def _lane_split(times: list[float]) -> tuple[int, list[int]]:
    """The side-stream split of _lanes for class times sorted longest first:
    the first class stays on the caller's stream; returns the number of side
    streams (1 to 3) and, for each later class, the side stream it joins (the
    least loaded so far).  The fewest side streams whose loads all fit within
    the first class's time; three when none does."""
    rest = times[1:]
    for n_side in range(1, min(3, len(rest)) + 1):
        load = [0.0] * n_side
        pick = []
        for t in rest:
            i = min(range(n_side), key=lambda j: load[j])
            load[i] += t
            pick.append(i)
        if max(load) <= times[0]:
            break
    return n_side, pick


class _Call:
    """One batched ``mamw_muon_step`` launch group (matrices of one shape class)."""

    __slots__ = ("device", "arr", "n", "ws_bytes", "m", "n_", "group")

    def __init__(self, device, arr, n, ws_bytes, m, n_, group):
        self.device, self.arr, self.n, self.ws_bytes, self.m, self.n_ = device, arr, n, ws_bytes, m, n_
        self.group = group  # index of the shape class (device, m, n)


class HipMuon:
    """Muon over a list of 2-D parameters, batched by shape on gfx950."""

    # Workspace per launch group is capped at this many bytes (None: 1/20 of
    # the device's memory, at most 16 GiB; on a 288 GB MI355X 14.4 GB, which
    # lets the 4096 x 14336 Llama-8B matrices run in groups of 32 whose
    # symmetric grids fill whole rounds of the 256 CUs: 3 ms per step faster
    # than groups of 20).  Within the cap, group_sizes() picks the split.
    workspace_limit_bytes: int | None = None
    # A step whose Newton-Schulz work (sum of ns_steps*(3 m^2 n + m^3)) is at
    # most this many flops runs its shape classes concurrently (lanes from
    # _lanes, one workspace per class): their launches are too small to fill
    # the GPU one after another (measured: GPT-2 Muon step -10%, config-3
    # -17%).  Larger steps run the classes in order, which keeps each class's
    # operands in the L2 and memory-side cache.  Measured on the first L
    # layers of the Llama-8B set, concurrent against in order: L = 1 (1.4e13)
    # 13.19 vs 14.10 ms, L = 2 (3.0e13) 26.46 vs 26.73, L = 4 (5.9e13) 52.72 vs
    # 52.10, L = 8 (1.2e14) 105.9 vs 102.9, all 32 layers 405 vs 391.
    concurrent_flops_limit = 4e13

    def __init__(
        self,
        params: Iterable[nn.Parameter] | list[nn.Parameter],
        lr: float = 1e-3,
        weight_decay: float = 0.1,
        coeffs: tuple[float, float, float] = (3.445, -4.775, 2.0315),
        nesterov: bool = True,
        beta: float = 0.95,
        ns_steps: int = 5,
        eps: float = 1e-7,
        adjust_lr_fn: Literal["original", "match_rms_adamw", "spectral_unclamped"] = "original",
    ):
        if adjust_lr_fn not in _ADJUST_FNS:
            raise AssertionError(f"Invalid adjust_lr_fn: {adjust_lr_fn}")
        self.model_params = list(params)
        self.a = coeffs[0]
        self.b = coeffs[1]
        self.c = coeffs[2]
        self.is_nesterov = nesterov
        self.beta = beta
        self.lr = lr
        self.adjust_lr_fn = adjust_lr_fn
        self.weight_decay = weight_decay
        self.steps = ns_steps
        self.eps = eps
        self.momentum = {}
        for param in self.model_params:
            self._momentum(param)
        self._plan_key = None
        self._plan_lr = lr
        self._calls: list[_Call] = []
        self._ws: dict = {}  # device (in order) or (device, shape class) (concurrent) -> workspace
        self._concurrent = False
        self._lanes: dict = {}  # (device, shape class) -> side stream, or None: the caller's stream

    def _momentum(self, param: nn.Parameter) -> torch.Tensor:
        """The momentum buffer of ``param``, created (zero) on first use: at
        construction, or for a parameter that joined ``model_params`` later
        (a parameter list loaded in the reference's state format).  fp32 also
        for bf16 parameters (the reference uses the parameter's dtype,
        :407-412)."""
        buf = self.momentum.get(param)
        if buf is None:
            buf = self.momentum[param] = torch.zeros_like(param, device=param.device, dtype=torch.float32)
        return buf

    def _build_calls(self, active: list[nn.Parameter]) -> None:
        groups: dict[tuple, list[nn.Parameter]] = {}
        for p in active:
            if p.ndim != 2:
                raise AssertionError("Muon only supports 2D tensors")
            g = p.grad
            _check_matrix(p, "param", bf16_ok=True)
            _check_matrix(g, "param.grad", bf16_ok=True)
            if g.shape != p.shape or g.device != p.device:
                raise ValueError("param.grad must match the parameter's shape and device")
            _check_matrix(self._momentum(p), "momentum")
            if self.momentum[p].shape != p.shape:
                raise ValueError(f"momentum buffer of shape {tuple(self.momentum[p].shape)} for a parameter of "
                                 f"shape {tuple(p.shape)}")
            R, C = p.shape
            groups.setdefault((p.device, min(R, C), max(R, C)), []).append(p)
        calls = []
        flops = sum(self.steps * (3.0 * m * m * n + float(m) ** 3) * len(pl) for (_, m, n), pl in groups.items())
        concurrent = len(groups) > 1 and flops <= self.concurrent_flops_limit
        need: dict = {}
        for gi, ((dev, m, n), plist) in enumerate(groups.items()):
            one = _workspace_bytes(1, m, n, self.steps)
            limit = self.workspace_limit_bytes
            if limit is None:
                limit = min(16 << 30, torch.cuda.get_device_properties(dev).total_memory // 20)
            cap = max(1, min(_lib.MUON_MAX_BATCH, limit // max(one, 1)))
            cus = torch.cuda.get_device_properties(dev).multi_processor_count
            sizes = iter(group_sizes(len(plist), cap, m, n, cus))
            per = next(sizes)
            chunks, cur, seen = [], [], set()
            for p in plist:  # a parameter listed twice goes to a later launch (launches are ordered)
                if len(cur) == per or id(p) in seen:
                    chunks.append(cur)
                    cur, seen = [], set()
                    per = next(sizes, per)
                cur.append(p)
                seen.add(id(p))
            chunks.append(cur)
            for chunk in chunks:
                arr = (_lib.MuonMatrix * len(chunk))()
                for i, p in enumerate(chunk):
                    R, C = p.shape
                    flags = (_lib.dtype_flag(p, _lib.BF16_PARAM, "param")
                             | _lib.dtype_flag(p.grad, _lib.BF16_GRAD, "param.grad"))
                    arr[i] = _lib.MuonMatrix(p.data_ptr(), p.grad.data_ptr(), self.momentum[p].data_ptr(), None,
                                             R, C, scaled_lr(self.lr, self.adjust_lr_fn, R, C), flags)
                wsb = _workspace_bytes(len(chunk), m, n, self.steps)
                calls.append(_Call(dev, arr, len(chunk), wsb, m, n, gi))
                key = (dev, gi) if concurrent else dev
                need[key] = max(need.get(key, 0), wsb)
        for key in [k for k in self._ws if k not in need]:
            del self._ws[key]
        for key, nbytes in need.items():
            ws = self._ws.get(key)
            if ws is None or ws.numel() < nbytes:
                self._ws[key] = None
                self._ws[key] = torch.empty(nbytes, dtype=torch.uint8, device=key[0] if concurrent else key)
        self._lanes = {}
        if concurrent:  # longest class first; a class's own launches keep their order (stable sort)
            cus = {d: torch.cuda.get_device_properties(d).multi_processor_count for d in dict.fromkeys(c.device for c in calls)}
            self._lanes, times = _lanes(calls, self.steps, cus)
            calls.sort(key=lambda c: -times[(c.device, c.group)])
        self._calls = calls
        self._concurrent = concurrent

    @torch.no_grad()
    def step(self):
        """Optimizer step for the Muon optimizer."""
        self._run(self._plan(), None, None)

    @torch.no_grad()
    def _step_amp(self, grad_scale: torch.Tensor | None, found_inf: torch.Tensor | None) -> None:
        """One step driven by ``torch.amp.GradScaler`` with its tensors left on the
        device: gradients divided by ``grad_scale``; where ``found_inf`` is
        non-zero the momentum and the parameters are left untouched (no host
        synchronisation).  Gradients are read, not rewritten."""
        self._run(self._plan(), grad_scale, found_inf)

    def _plan(self) -> list[nn.Parameter]:
        """The parameters that have a gradient, with the launch plan checked
        (rebuilt when any of them changed): argument errors raise here, before
        anything of the step is queued."""
        active = [p for p in self.model_params if p.grad is not None]
        if not active:
            return active
        key = (self.adjust_lr_fn, self.steps, tuple(_lib.layout_key(p) for p in active))
        if key != self._plan_key:
            _lib.check_not_capturing("Muon")
            self._plan_key = None
            self._build_calls(active)
            self._plan_key = key
            self._plan_lr = self.lr
        elif self.lr != self._plan_lr:  # a schedule moved lr: refresh the per-matrix scaled lr only
            for call in self._calls:
                for i in range(call.n):
                    e = call.arr[i]
                    e.scaled_lr = scaled_lr(self.lr, self.adjust_lr_fn, e.rows, e.cols)
            self._plan_lr = self.lr
        return active

    def _run(self, active: list[nn.Parameter], grad_scale: torch.Tensor | None,
             found_inf: torch.Tensor | None) -> None:
        """Queue the step over ``active`` (planned by :meth:`_plan`)."""
        if not active:
            return
        lib = _lib.load()
        nest = int(bool(self.is_nesterov))

        amp = grad_scale is not None or found_inf is not None
        amp_ptrs: dict = {}  # device -> (grad_scale, found_inf) on that device, made before any fork
        if amp:
            for call in self._calls:
                if call.device not in amp_ptrs:
                    amp_ptrs[call.device] = tuple(
                        t.to(call.device, torch.float32, non_blocking=True) if t is not None else None
                        for t in (grad_scale, found_inf))

        def launch(call, ws, stream_handle):
            with torch.cuda.device(call.device):
                if not amp:
                    st = lib.mamw_muon_step(call.arr, call.n, self.lr, self.weight_decay, self.beta, nest,
                                            self.a, self.b, self.c, self.steps, self.eps, ws.data_ptr(),
                                            ws.numel(), stream_handle)
                else:
                    gs, fi = amp_ptrs[call.device]
                    st = lib.mamw_muon_step_amp(call.arr, call.n, self.lr, self.weight_decay, self.beta, nest,
                                                self.a, self.b, self.c, self.steps, self.eps, ws.data_ptr(),
                                                ws.numel(), gs.data_ptr() if gs is not None else None,
                                                fi.data_ptr() if fi is not None else None, stream_handle)
            _lib.check(st, "mamw_muon_step")

        if not self._concurrent:
            for call in self._calls:
                ws, cur = self._ws[call.device], torch.cuda.current_stream(call.device)
                ws.record_stream(cur)  # allocated under the stream current when the plan was built
                launch(call, ws, cur.cuda_stream)
            return
        # Concurrent shape classes (lanes from _lanes): the largest on the
        # caller's current stream, the others on side streams.  Every side
        # stream waits for the caller's stream before anything of this step is
        # queued there, runs its classes' launches in order, and the caller's
        # stream waits for all of them at the end, so the step stays ordered
        # with the caller's work on its stream.
        side = {}
        for call in self._calls:
            s = self._lanes[(call.device, call.group)]
            if s is not None and (call.device, id(s)) not in side:
                side[(call.device, id(s))] = s
                s.wait_stream(torch.cuda.current_stream(call.device))
                for t in amp_ptrs.get(call.device, ()):  # the scaler may drop its tensors after step()
                    if t is not None:
                        t.record_stream(s)
        for call in self._calls:
            key = (call.device, call.group)
            s = self._lanes[key]
            if s is None:
                s = torch.cuda.current_stream(call.device)
            self._ws[key].record_stream(s)
            launch(call, self._ws[key], s.cuda_stream)
        for (dev, _), s in side.items():
            torch.cuda.current_stream(dev).wait_stream(s)

    def zero_grad(self, set_to_none: bool = False):
        """Resets gradients back to zero (the reference's behaviour), or to None
        with ``set_to_none=True`` (torch.optim's)."""
        for param in self.model_params:
            if param.grad is not None:
                if set_to_none:
                    param.grad = None
                else:
                    param.grad.zero_()

    def state_dict(self) -> dict:
        """Optimizer state in ``torch.optim.Muon``'s format: ``state[i]`` holds the
        ``momentum_buffer`` of parameter ``i`` (its position in ``model_params``),
        returned by reference; one param group with this branch's
        hyperparameters (``adjust_lr_fn`` ``"original"`` written as torch's
        ``None``)."""
        state = {i: {"momentum_buffer": self._momentum(p)} for i, p in enumerate(self.model_params)}
        group = {"lr": self.lr, "weight_decay": self.weight_decay, "momentum": self.beta,
                 "nesterov": self.is_nesterov, "ns_coefficients": (self.a, self.b, self.c), "eps": self.eps,
                 "ns_steps": self.steps,
                 "adjust_lr_fn": None if self.adjust_lr_fn == "original" else self.adjust_lr_fn,
                 "params": list(range(len(self.model_params)))}
        return {"state": state, "param_groups": [group]}

    def load_state_dict(self, state_dict: dict) -> None:
        """Restore a state produced by :meth:`state_dict` or by ``torch.optim.Muon``.

        Parameters are matched by position; momentum buffers are copied into
        this branch's own (parameters without saved state restart from zero,
        as torch's lazily created buffers do).
        """
        groups = state_dict["param_groups"]
        ids = [i for g in groups for i in g["params"]]
        if len(ids) != len(self.model_params):
            raise ValueError("loaded state dict contains a parameter group that doesn't match the size of "
                             "optimizer's group")
        keys = ("lr", "weight_decay", "momentum", "nesterov", "ns_coefficients", "eps", "ns_steps", "adjust_lr_fn")
        hyper = {tuple(tuple(g[k]) if k == "ns_coefficients" else g[k] for k in keys) for g in groups}
        if len(hyper) > 1:
            raise ValueError("parameter groups with different hyperparameters cannot be loaded into one Muon branch")
        pos = {pid: k for k, pid in enumerate(ids)}
        with torch.no_grad():
            for p in self.model_params:
                self._momentum(p).zero_()
            for pid, st in state_dict["state"].items():
                self._momentum(self.model_params[pos[pid]]).copy_(st["momentum_buffer"])
        if hyper:
            lr, wd, beta, nesterov, coeffs, eps, steps, adjust = hyper.pop()
            adjust = "original" if adjust is None else adjust
            if adjust not in _ADJUST_FNS:
                raise AssertionError(f"Invalid adjust_lr_fn: {adjust}")
            self.lr, self.weight_decay, self.beta, self.is_nesterov = lr, wd, beta, nesterov
            self.a, self.b, self.c = coeffs
            self.eps, self.steps, self.adjust_lr_fn = eps, steps, adjust


# The reference's class name, for drop-in imports.
TritonMuon = HipMuon
