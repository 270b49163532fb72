"""AdamW branch on the gfx950 multi-tensor kernel.

Drop-in for the reference's ``TritonAdamW`` (adamw/triton_adam.py:106-161) and
``solve_adamw_step`` (:66-103): same constructor, attributes (``model_params``,
``beta1``, ``beta2``, ``lr``, ``weight_decay``, ``eps``, ``step_num``, ``m``,
``v``) and step semantics:

* one global ``step_num``, incremented on every ``step()`` call, also for
  parameters whose gradient is ``None`` (triton_adam.py:137);
* bias corrections ``1 - beta**step_num`` computed on the host in float64 and
  handed to the kernel as float32 (:147-148);
* parameters whose ``grad`` is ``None`` are skipped (:139-140);
* ``zero_grad()`` zero-fills existing gradients (:155-161).

Where the reference launches one kernel per parameter, ``step()`` launches
one kernel for all of them (``mamw_adamw_mt_step``).  The packed tensor table
lives in device memory and is rebuilt only when a parameter or gradient
pointer changes.  Parameters may have any number of dimensions (the reference
handles 1-D and 2-D only); they must be contiguous on a ROCm device, float32
or bfloat16 (parameters and gradients independently), with fp32 moments in
every case: a bf16 parameter is updated in fp32 and rounded back to
nearest-even (no counterpart in the reference, whose kernel runs in the
parameter's dtype, triton_adam.py:79-85).
"""

from __future__ import annotations

import ctypes
from collections.abc import Iterable

import torch
import torch.nn as nn

from .. import _lib


def _check_tensor(t: torch.Tensor, name: str, bf16_ok: bool = False) -> None:
    _lib.require_gpu_tensor(t, name)
    if t.dtype != torch.float32 and not (bf16_ok and t.dtype == torch.bfloat16):
        raise TypeError(f"{name} must be float32{' or bfloat16' if bf16_ok else ''} (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def solve_adamw_step(matrix: torch.Tensor, gradient: torch.Tensor, m: torch.Tensor, v: torch.Tensor,
                     lr: float, bias1: float, bias2: float, beta1: float, beta2: float,
                     weight_decay: float, eps: float) -> None:
    """One AdamW update of one tensor in place (triton_adam.py:66-103)."""
    for t, name in ((matrix, "param"), (gradient, "grad"), (m, "exp_avg"), (v, "exp_avg_sq")):
        _check_tensor(t, name)
        if t.numel() != matrix.numel() or t.device != matrix.device:
            raise ValueError(f"{name} must match the parameter's numel and device")
    lib = _lib.load()
    with torch.cuda.device(matrix.device):
        st = lib.mamw_adamw_tensor_step(
            matrix.data_ptr(), gradient.data_ptr(), m.data_ptr(), v.data_ptr(), matrix.numel(),
            lr, bias1, bias2, beta1, beta2, weight_decay, eps, _lib.stream_handle(matrix.device))
    _lib.check(st, "mamw_adamw_tensor_step")


class _DevicePlan:
    """Packed tensor table of one device, resident in device memory."""

    __slots__ = ("device", "table", "n_tensors", "n_blocks")

    def __init__(self, device: torch.device, entries: list[tuple[torch.Tensor, ...]]):
        lib = _lib.load()
        n = len(entries)
        arr = (_lib.AdamWTensorEx * n)()
        for i, (p, g, m, v) in enumerate(entries):
            flags = _lib.dtype_flag(p, _lib.BF16_PARAM, "param") | _lib.dtype_flag(g, _lib.BF16_GRAD, "param.grad")
            arr[i] = _lib.AdamWTensorEx(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), p.numel(), flags, 0)
        nbytes = ctypes.c_size_t()
        _lib.check(lib.mamw_adamw_table_bytes(n, ctypes.byref(nbytes)), "mamw_adamw_table_bytes")
        # Packed into pinned memory and copied without blocking the host: the
        # table is rebuilt whenever a gradient tensor is replaced (every step
        # under zero_grad(set_to_none=True)), and a pageable upload would
        # synchronise each time.  torch's pinned-memory allocator keeps the
        # staging block until the copy has completed.
        host = torch.empty(max(nbytes.value, 1), dtype=torch.uint8, pin_memory=True)
        nblocks = ctypes.c_int64()
        _lib.check(lib.mamw_adamw_table_pack_ex(arr, n, host.data_ptr(), nbytes.value, ctypes.byref(nblocks)),
                   "mamw_adamw_table_pack_ex")
        self.device = device
        self.table = torch.empty(host.numel(), dtype=torch.uint8, device=device)
        with torch.cuda.device(device):
            self.table.copy_(host, non_blocking=True)
        self.n_tensors = n
        self.n_blocks = nblocks.value

    def launch_stream(self) -> int:
        """Handle of the current stream, on which the table is about to be
        read.  The table was allocated on the stream current when it was packed;
        recording this one keeps torch's allocator from reusing the table's
        memory, once the plan is replaced, before the launch has run."""
        s = torch.cuda.current_stream(self.device)
        self.table.record_stream(s)
        return s.cuda_stream


class HipAdamW:
    """AdamW over a list of parameters, one gfx950 kernel launch per step.

    ``capturable=True`` (as in torch.optim.AdamW) keeps the step counter on the
    device from the first step on, so that a step captured in a CUDA/HIP graph
    advances it, and forms the bias corrections from it, at every replay.
    """

    def __init__(
        self,
        params: Iterable[nn.Parameter] | list[nn.Parameter],
        lr=1e-3,
        betas: tuple[float, float] = (0.9, 0.999),
        weight_decay=1e-2,
        eps=1e-7,
        *,
        capturable: bool = False,
    ):
        self.capturable = bool(capturable)
        self.model_params = list(params)
        self.beta1 = betas[0]
        self.beta2 = betas[1]
        self.lr = lr
        self.weight_decay = weight_decay
        self.eps = eps
        self.step_num = 0  # also creates the (empty) device-side counters, see step_num
        self.m = {}
        self.v = {}
        for param in self.model_params:
            self._moments(param)
        self._plan_key = None
        self._plans: list[_DevicePlan] = []

    def _moments(self, param: nn.Parameter) -> tuple[torch.Tensor, torch.Tensor]:
        """``(exp_avg, exp_avg_sq)`` of ``param``, created (zero, fp32) on first
        use: at construction, or for a parameter that joined ``model_params``
        later (a parameter list loaded in the reference's state format)."""
        m = self.m.get(param)
        if m is None:
            m = self.m[param] = torch.zeros_like(param, dtype=torch.float32)
            self.v[param] = torch.zeros_like(param, dtype=torch.float32)
        return m, self.v[param]

    def _build_plans(self, active: list[nn.Parameter]) -> None:
        # A parameter listed k times is updated k times in sequence, as the
        # reference's per-parameter loop does (triton_adam.py:138-153): its
        # i-th occurrence goes to launch pass i (one table per pass and
        # device; a table may hold a tensor only once).
        passes: list[dict[torch.device, list]] = []
        seen: dict[int, int] = {}
        for p in active:
            g = p.grad
            _check_tensor(p, "param", bf16_ok=True)
            _check_tensor(g, "param.grad", bf16_ok=True)
            if g.shape != p.shape or g.device != p.device:
                raise ValueError("param.grad must match the parameter's shape and device")
            m, v = self._moments(p)
            _check_tensor(m, "exp_avg")
            _check_tensor(v, "exp_avg_sq")
            if m.shape != p.shape or v.shape != p.shape:
                raise ValueError(f"moments of shape {tuple(m.shape)} / {tuple(v.shape)} for a parameter of "
                                 f"shape {tuple(p.shape)}")
            k = seen[id(p)] = seen.get(id(p), -1) + 1
            if k == len(passes):
                passes.append({})
            passes[k].setdefault(p.device, []).append((p, g, m, v))
        self._plans = [_DevicePlan(dev, ents) for by_dev in passes for dev, ents in by_dev.items()]

    @property
    def step_num(self) -> int:
        """The global step counter (triton_adam.py:137).  After a gradient-scaler
        step (``_step_amp``) it lives on the device, one fp32 counter per device
        as torch's fused AdamW keeps it; reading it then synchronises."""
        if self._dev_steps:
            return int(next(iter(self._dev_steps.values())).item())
        return self._step_host

    @step_num.setter
    def step_num(self, value: int) -> None:
        """Set the counter.  Once device-side counters exist they are filled in
        place and kept: a step captured in a graph writes to those very
        tensors, so replacing them would leave the graph advancing freed
        memory while the bias corrections ignored the new value."""
        self._step_host = int(value)
        devs = getattr(self, "_dev_steps", None)
        if devs:
            with torch.no_grad():
                for c in devs.values():
                    c.fill_(float(value))
        else:
            self._dev_steps: dict[torch.device, torch.Tensor] = {}

    def _refresh_plans(self, active: list[nn.Parameter]) -> None:
        key = tuple(_lib.layout_key(p) for p in active)
        if key != self._plan_key:
            _lib.check_not_capturing("AdamW")
            self._plan_key = None
            self._build_plans(active)
            self._plan_key = key

    def _plan(self) -> list[nn.Parameter]:
        """The parameters that have a gradient, with their launch plan checked
        (rebuilt when any of them changed): argument errors raise here, before
        anything of the step is queued or counted."""
        active = [p for p in self.model_params if p.grad is not None]
        if active:
            self._refresh_plans(active)
        return active

    @torch.no_grad()
    def step(self):
        """Performs one iteration of the AdamW optimizer step."""
        self._launch(self._plan(), None, None)

    @torch.no_grad()
    def _step_amp(self, grad_scale: torch.Tensor | None, found_inf: torch.Tensor | None) -> None:
        """One step driven by ``torch.amp.GradScaler`` with its tensors left on
        the device, as torch's fused AdamW takes them (torch/optim/adam.py:865-899):
        gradients divided by ``grad_scale``, no update where ``found_inf`` is
        non-zero, and the step counter incremented before the launch and
        decremented by ``found_inf`` after it, on the device.  Gradients are
        read, not rewritten."""
        self._launch(self._plan(), grad_scale, found_inf, amp=True)

    def _launch(self, active: list[nn.Parameter], grad_scale: torch.Tensor | None,
                found_inf: torch.Tensor | None, amp: bool = False) -> None:
        """Queue the step over ``active`` (planned by :meth:`_plan`)."""
        if not amp and (self.capturable or self._dev_steps):
            # The counter lives on the device (capturable, or after a gradient-
            # scaler step): keep it there, so that no step reads it back.
            amp = True
        if not amp:
            self.step_num += 1
            if not active:
                return
            lib = _lib.load()
            bias1 = 1 - self.beta1**self._step_host
            bias2 = 1 - self.beta2**self._step_host
            for plan in self._plans:
                with torch.cuda.device(plan.device):
                    st = lib.mamw_adamw_mt_step(
                        plan.table.data_ptr(), plan.n_tensors, plan.n_blocks, self.lr, bias1, bias2,
                        self.beta1, self.beta2, self.weight_decay, self.eps, plan.launch_stream())
                _lib.check(st, "mamw_adamw_mt_step")
            return
        if not active:  # nothing to update: the counter alone
            if self._dev_steps:
                for c in self._dev_steps.values():
                    c.add_(1.0)
                    if found_inf is not None:
                        c.sub_(found_inf.to(c.device, torch.float32, non_blocking=True))
            elif found_inf is None or float(found_inf) == 0.0:
                self._step_host += 1
            return
        lib = _lib.load()
        if not self._dev_steps:
            _lib.check_not_capturing("AdamW")
            start = float(self._step_host)
            self._dev_steps = {plan.device: torch.full((), start, dtype=torch.float32, device=plan.device)
                               for plan in self._plans}
        # Per device: the counter advances once, every pass of the step reads
        # it, and a skipped step takes it back once.
        scaler: dict = {}
        for dev in dict.fromkeys(plan.device for plan in self._plans):
            if dev not in self._dev_steps:
                self._dev_steps[dev] = next(iter(self._dev_steps.values())).to(dev)
            gs = grad_scale.to(dev, torch.float32, non_blocking=True) if grad_scale is not None else None
            fi = found_inf.to(dev, torch.float32, non_blocking=True) if found_inf is not None else None
            scaler[dev] = (gs, fi)
            with torch.cuda.device(dev):
                self._dev_steps[dev].add_(1.0)
        for plan in self._plans:
            dev = plan.device
            gs, fi = scaler[dev]
            with torch.cuda.device(dev):
                st = lib.mamw_adamw_mt_step_amp(
                    plan.table.data_ptr(), plan.n_tensors, plan.n_blocks, self.lr, self.beta1, self.beta2,
                    self.weight_decay, self.eps, self._dev_steps[dev].data_ptr(),
                    gs.data_ptr() if gs is not None else None, fi.data_ptr() if fi is not None else None,
                    plan.launch_stream())
            _lib.check(st, "mamw_adamw_mt_step_amp")
        for dev, (_, fi) in scaler.items():
            if fi is not None:
                with torch.cuda.device(dev):
                    self._dev_steps[dev].sub_(fi)

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
        """Optimizer state in ``torch.optim.AdamW``'s format.

        ``state[i]`` holds ``exp_avg``, ``exp_avg_sq`` and ``step`` of parameter
        ``i`` (its position in ``model_params``); every parameter carries the
        branch's one step counter (triton_adam.py:137).  Empty before the first
        step, as in torch.  The state tensors are returned by reference.
        """
        state = {}
        if self.step_num > 0:
            for i, p in enumerate(self.model_params):
                m, v = self._moments(p)
                state[i] = {"step": torch.tensor(float(self.step_num)), "exp_avg": m, "exp_avg_sq": v}
        group = {"lr": self.lr, "betas": (self.beta1, self.beta2), "eps": self.eps,
                 "weight_decay": self.weight_decay, "amsgrad": False, "maximize": False, "foreach": None,
                 "capturable": self.capturable, "differentiable": False, "fused": True, "decoupled_weight_decay": True,
                 "params": list(range(len(self.model_params)))}
        return {"state": state, "param_groups": [group]}

    def load_state_dict(self, state_dict: dict) -> None:
        """Restore a state produced by :meth:`state_dict` or by ``torch.optim.AdamW``.

        Parameters are matched by position; the moments are copied into this
        branch's own buffers (so the launch plan stays valid).  torch keeps one
        step per parameter, this branch one for all: differing steps raise.
        """
        groups = state_dict["param_groups"]
        ids = [i for g in groups for i in g["params"]]
        if len(ids) != len(self.model_params):
            raise ValueError("loaded state dict contains a parameter group that doesn't match the size of "
                             "optimizer's group")
        hyper = {(g["lr"], tuple(g["betas"]), g["eps"], g["weight_decay"]) for g in groups}
        if len(hyper) > 1:
            raise ValueError("parameter groups with different hyperparameters cannot be loaded into one AdamW branch")
        pos = {pid: k for k, pid in enumerate(ids)}
        steps = {float(st["step"]) for st in state_dict["state"].values()}
        if len(steps) > 1:
            raise ValueError(f"per-parameter steps differ ({sorted(steps)}); this optimizer keeps one step counter")
        with torch.no_grad():
            for p in self.model_params:
                for t in self._moments(p):
                    t.zero_()
            for pid, st in state_dict["state"].items():
                m, v = self._moments(self.model_params[pos[pid]])
                m.copy_(st["exp_avg"])
                v.copy_(st["exp_avg_sq"])
        self.step_num = int(steps.pop()) if steps else 0
        lr, betas, eps, wd = hyper.pop() if hyper else (self.lr, (self.beta1, self.beta2), self.eps, self.weight_decay)
        self.lr, self.beta1, self.beta2, self.eps, self.weight_decay = lr, betas[0], betas[1], eps, wd


# The reference's class name, for drop-in imports.
TritonAdamW = HipAdamW
