"""The hybrid MuonAdamW optimizer and its configuration (drop-in API).

Mirrors ``MuonAdamW package/triton_muon_adamw/optimizer.py``:

* ``AdamConfig`` / ``MuonConfig`` (:14-67): same fields and defaults;
* ``MuonAdamW`` (:70-175): same constructor (argument order
  ``model_params, muon_config, adam_config, parameter_split``), the same
  ``auto`` / ``explicit`` routing and errors (:107-130), ``.adamw``,
  ``.muon`` and ``.param_group`` attributes, ``step`` = AdamW branch then
  Muon branch on the current stream with no host synchronisation,
  zero-filling ``zero_grad``, and ``state_dict`` / ``load_state_dict``
  carrying the parameter lists (:166-175);
* ``PyTorchMuonAdamW`` (:178-260): the torch.optim wrapper the reference
  checks itself against (fused ``torch.optim.AdamW`` + ``torch.optim.Muon``).

The branches run on gfx950 HIP kernels (``adamw.HipAdamW``, ``muon.HipMuon``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal, TypeAlias

import torch
import torch.nn as nn

from .adamw.hip_adam import HipAdamW
from .muon.hip_muon import _ADJUST_FNS, HipMuon

ParameterGroups: TypeAlias = dict[str, list[nn.Parameter]]


@dataclass
class AdamConfig:
    """Settings of the elementwise branch (every parameter that is not a
    Muon matrix).

    ``lr`` is the AdamW step size.  ``betas`` = (decay of the gradient mean,
    decay of the squared-gradient mean).  ``eps`` is added to
    ``sqrt(v_hat)`` before the division, so a tensor whose second moment is
    still zero gets a finite step.  ``weight_decay`` shrinks the parameter by
    ``lr * weight_decay`` each step, outside the adaptive term.
    """

    lr: float = 1e-3
    betas: tuple[float, float] = (0.9, 0.999)
    eps: float = 1e-7
    weight_decay: float = 0.01


@dataclass
class MuonConfig:
    """Settings of the matrix branch (orthogonalised momentum updates).

    ``lr`` is the base step size; ``adjust_lr_fn`` picks how it is rescaled by
    the matrix shape (``"original"``: ``sqrt(max(1, rows/cols))``,
    ``"match_rms_adamw"``: ``0.2 * sqrt(max(rows, cols))``,
    ``"spectral_unclamped"``: ``sqrt(rows/cols)``).  ``beta`` is the momentum
    decay and ``nesterov`` selects the look-ahead blend of gradient and
    momentum.  ``eps`` floors the Frobenius norm the momentum is divided by
    before the iteration.  ``weight_decay`` multiplies the unscaled ``lr``.
    ``coeffs`` = (a, b, c) of the quintic ``aX + b(XX^T)X + c(XX^T)^2 X`` that
    is applied ``ns_steps`` times.
    """

    lr: float = 1e-3
    beta: float = 0.95
    eps: float = 1e-7
    weight_decay: float = 0.1
    coeffs: tuple[float, float, float] = (3.445, -4.775, 2.0315)
    nesterov: bool = True
    ns_steps: int = 5
    adjust_lr_fn: Literal["original", "match_rms_adamw", "spectral_unclamped"] = "original"


def split_parameters(
    model_params: nn.Module | ParameterGroups,
    parameter_split: Literal["auto", "explicit"] = "auto",
) -> tuple[list[nn.Parameter], list[nn.Parameter]]:
    """Route parameters to (adam, muon) lists exactly as optimizer.py:105-130.

    ``explicit``: ``model_params["adam"]`` and ``model_params["muon"]`` (each
    defaulting to ``[]``).  ``auto``: walk ``model_params.parameters()``,
    skipping frozen parameters and storage already seen (``data_ptr`` dedupe);
    2-D parameters go to Muon unless they are the input embedding or output
    head weight; everything else goes to AdamW.
    """
    adam_params: list[nn.Parameter] = []
    muon_params: list[nn.Parameter] = []
    if parameter_split == "explicit" and not isinstance(model_params, dict):
        raise ValueError(
            "When parameter_split is 'explicit', params must be a dictionary with keys 'adam' and 'muon' "
            "and their corresponding parameters.")
    if parameter_split == "auto" and isinstance(model_params, dict):
        raise ValueError(
            "When parameter_split is 'auto', params must be an nn.Module (ie the model itself), "
            "not a dictionary.")
    if parameter_split == "explicit":
        adam_params = model_params.get("adam", [])
        muon_params = model_params.get("muon", [])
    elif parameter_split == "auto":
        embed = model_params.get_input_embeddings().weight
        head_mod = model_params.get_output_embeddings()
        head = head_mod.weight if head_mod is not None else None
        seen_ptrs = set()
        for p in model_params.parameters():
            if not p.requires_grad or p.data_ptr() in seen_ptrs:
                continue
            seen_ptrs.add(p.data_ptr())
            if p.ndim == 2 and p is not embed and p is not head:
                muon_params.append(p)
            else:
                adam_params.append(p)
    return adam_params, muon_params


class MuonAdamW(HipMuon, HipAdamW, torch.optim.Optimizer):
    """Hybrid optimizer: Muon for 2-D weight matrices, AdamW for the rest.

    The Muon branch takes the weight matrices (every 2-D parameter other
    than the token embedding and the LM head); the AdamW branch takes what is
    left: vectors such as biases and norm gains, and the embedding and head
    matrices themselves.

    Parameters
    ----------
    model_params:
        The model (``parameter_split="auto"``; it must provide
        ``get_input_embeddings()`` and ``get_output_embeddings()``), or a
        dictionary with ``"adam"`` and ``"muon"`` parameter lists
        (``parameter_split="explicit"``).
    muon_config:
        Hyperparameters of the Muon branch.
    adam_config:
        Hyperparameters of the AdamW branch.
    parameter_split:
        ``"auto"`` or ``"explicit"``.

    Notes
    -----
    The update kernels are gfx950 HIP kernels; parameters must be contiguous
    float32 tensors on a ROCm device when ``step()`` runs.

    Beyond the reference's surface, the optimizer is a ``torch.optim.Optimizer``
    with two ``param_groups`` (0: the AdamW branch, 1: the Muon branch, with
    torch.optim.AdamW / torch.optim.Muon hyperparameter names), so LR schedulers
    attach and hyperparameters edited there take effect at the next ``step``;
    ``step(closure)`` re-evaluates the loss first; ``zero_grad(set_to_none)``;
    and ``state_dict()`` carries the optimizer state (moments, step, momentum)
    in the format of ``PyTorchMuonAdamW.state_dict()``, so checkpoints move
    between the two in both directions.

    ``capturable=True`` (keyword only, as torch.optim.AdamW's flag) lets a step
    be captured in a CUDA/HIP graph (``torch.cuda.graph``) after one eager step:
    the AdamW step counter lives on the device and advances at every replay.
    A replay reuses the launches recorded at capture: the parameter, gradient
    and state tensors (copy new gradients into the same ``.grad`` tensors) and
    the hyperparameters of that moment (learning rates included).
    """

    # torch.amp.GradScaler passes grad_scale / found_inf to step() instead of
    # unscaling in place and reading found_inf on the host.
    _step_supports_amp_scaling = True

    def __init__(
        self,
        model_params: nn.Module | ParameterGroups,
        muon_config: MuonConfig = MuonConfig(),  # noqa: B008
        adam_config: AdamConfig = AdamConfig(),  # noqa: B008
        parameter_split: Literal["auto", "explicit"] = "auto",
        *,
        capturable: bool = False,
    ) -> None:
        adam_params, muon_params = split_parameters(model_params, parameter_split)
        self.adamw = HipAdamW(
            params=adam_params,
            lr=adam_config.lr,
            betas=adam_config.betas,
            weight_decay=adam_config.weight_decay,
            eps=adam_config.eps,
            capturable=capturable,
        )
        self.muon = HipMuon(
            params=muon_params,
            lr=muon_config.lr,
            beta=muon_config.beta,
            eps=muon_config.eps,
            weight_decay=muon_config.weight_decay,
            coeffs=muon_config.coeffs,
            nesterov=muon_config.nesterov,
            ns_steps=muon_config.ns_steps,
            adjust_lr_fn=muon_config.adjust_lr_fn,
        )
        self.param_group = {
            "adam": self.adamw.model_params,
            "muon": self.muon.model_params,
        }
        torch.optim.Optimizer.__init__(self, [self._adam_group(), self._muon_group()], {})
        self._push_groups()  # the groups share the branches' parameter lists
        self._groups_fixed = True

    # -- torch.optim surface ---------------------------------------------------
    def add_param_group(self, param_group: dict) -> None:
        """Only at construction: the two groups ("adam", "muon") are the two
        branches.  Later, a parameter joins a branch through its list
        (``param_group["adam"]`` / ``["muon"]``, as in the reference)."""
        if getattr(self, "_groups_fixed", False):
            raise ValueError("MuonAdamW has two fixed parameter groups ('adam' and 'muon'); append parameters to "
                             "param_group['adam'] or param_group['muon'] instead of add_param_group")
        super().add_param_group(param_group)

    def _adam_group(self) -> dict:
        a = self.adamw
        return {"params": a.model_params, "lr": a.lr, "betas": (a.beta1, a.beta2), "eps": a.eps,
                "weight_decay": a.weight_decay, "name": "adam"}

    def _muon_group(self) -> dict:
        m = self.muon
        return {"params": m.model_params, "lr": m.lr, "momentum": m.beta, "nesterov": m.is_nesterov,
                "ns_coefficients": (m.a, m.b, m.c), "eps": m.eps, "ns_steps": m.steps,
                "weight_decay": m.weight_decay, "adjust_lr_fn": m.adjust_lr_fn, "name": "muon"}

    def _pull_groups(self) -> None:
        """Hyperparameters edited in ``param_groups`` (e.g. by a scheduler) into the branches."""
        ga, gm = self.param_groups
        a, m = self.adamw, self.muon
        a.lr, (a.beta1, a.beta2), a.eps, a.weight_decay = ga["lr"], ga["betas"], ga["eps"], ga["weight_decay"]
        m.lr, m.beta, m.is_nesterov, m.eps = gm["lr"], gm["momentum"], gm["nesterov"], gm["eps"]
        (m.a, m.b, m.c), m.steps, m.weight_decay = gm["ns_coefficients"], gm["ns_steps"], gm["weight_decay"]
        adjust = "original" if gm["adjust_lr_fn"] is None else gm["adjust_lr_fn"]  # torch's None
        if adjust not in _ADJUST_FNS:
            raise AssertionError(f"Invalid adjust_lr_fn: {adjust}")
        m.adjust_lr_fn = adjust

    def _push_groups(self) -> None:
        """The branches' hyperparameters (after a load) into ``param_groups``."""
        ga, gm = self.param_groups
        for g, new in ((ga, self._adam_group()), (gm, self._muon_group())):
            for k, v in new.items():
                if k != "params":
                    g[k] = v
        ga["params"], gm["params"] = self.adamw.model_params, self.muon.model_params

    def step(self, closure=None):
        """Apply one update with the AdamW branch, then the Muon branch.

        With ``closure``, the loss is re-evaluated (under ``torch.enable_grad``)
        before the update and returned, as torch.optim does.  Under
        ``torch.amp.GradScaler`` (``_step_supports_amp_scaling``) the scaler
        hands over ``grad_scale`` and ``found_inf`` as device tensors
        (torch/amp/grad_scaler.py:403-448): both branches unscale the gradients
        in their kernels and skip a non-finite step on the device, with no host
        synchronisation, as torch's fused AdamW does.
        """
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self._pull_groups()
        grad_scale = getattr(self, "grad_scale", None)
        found_inf = getattr(self, "found_inf", None)
        amp = grad_scale is not None or found_inf is not None
        with torch.no_grad():
            # Both branches' plans first: an invalid argument in either raises
            # before anything of the step is queued.
            adam_active, muon_active = self.adamw._plan(), self.muon._plan()
            self.adamw._launch(adam_active, grad_scale, found_inf, amp=amp)
            self.muon._run(muon_active, grad_scale, found_inf)
        return loss

    def zero_grad(self, set_to_none: bool = False) -> None:
        """Zero the gradients of every parameter of both branches (or set them
        to None with ``set_to_none=True``)."""
        self.adamw.zero_grad(set_to_none)
        self.muon.zero_grad(set_to_none)

    def state_dict(self) -> dict[str, object]:
        """Both branches' optimizer state, ``{"adam": <torch.optim.AdamW format>,
        "muon": <torch.optim.Muon format>}`` (the format of
        ``PyTorchMuonAdamW.state_dict()``).  The reference returned only the
        parameter lists (optimizer.py:166-168); those remain in ``param_group``."""
        self._pull_groups()
        return {"adam": self.adamw.state_dict(), "muon": self.muon.state_dict()}

    def load_state_dict(self, state_dict: dict[str, object]) -> None:
        """Load optimizer state from :meth:`state_dict` or ``PyTorchMuonAdamW.state_dict()``.

        A branch entry that is a list of parameters (the reference's format,
        optimizer.py:170-175) replaces that branch's parameter list instead.
        """
        if "adam" in state_dict:
            sd = state_dict["adam"]
            if isinstance(sd, dict):
                self.adamw.load_state_dict(sd)
            else:
                self.adamw.model_params = sd
                self.param_group["adam"] = sd
        if "muon" in state_dict:
            sd = state_dict["muon"]
            if isinstance(sd, dict):
                self.muon.load_state_dict(sd)
            else:
                self.muon.model_params = sd
                self.param_group["muon"] = sd
        self._push_groups()


class PyTorchMuonAdamW:
    """torch.optim reference implementation (optimizer.py:178-260).

    Same routing as :class:`MuonAdamW`; delegates to ``torch.optim.AdamW``
    (``fused=True``) and ``torch.optim.Muon``.  Unlike the reference wrapper,
    it forwards ``MuonConfig.coeffs`` and ``MuonConfig.eps`` to
    ``torch.optim.Muon`` (the reference drops them, :228-236, so its wrapper
    always ran torch's defaults); with torch's default coefficients the two
    are the same.  Runs on CPU or GPU tensors.
    """

    def __init__(
        self,
        model_params: nn.Module | ParameterGroups,
        muon_config: MuonConfig = MuonConfig(),  # noqa: B008
        adam_config: AdamConfig = AdamConfig(),  # noqa: B008
        parameter_split: Literal["auto", "explicit"] = "auto",
    ) -> None:
        adam_params, muon_params = split_parameters(model_params, parameter_split)
        self.adamw = torch.optim.AdamW(
            params=adam_params,
            lr=adam_config.lr,
            betas=adam_config.betas,
            weight_decay=adam_config.weight_decay,
            eps=adam_config.eps,
            fused=True,
        )
        self.muon = torch.optim.Muon(
            params=muon_params,
            lr=muon_config.lr,
            momentum=muon_config.beta,
            weight_decay=muon_config.weight_decay,
            nesterov=muon_config.nesterov,
            ns_coefficients=tuple(muon_config.coeffs),
            eps=muon_config.eps,
            ns_steps=muon_config.ns_steps,
            adjust_lr_fn=muon_config.adjust_lr_fn,
        )

    def step(self, closure=None):
        """torch's AdamW step, then torch's Muon step (``closure`` as torch.optim)."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self.adamw.step()
        self.muon.step()
        return loss

    def zero_grad(self, *args, **kwargs) -> None:
        """Clear the gradients of both torch optimizers (torch's default: set to None)."""
        self.adamw.zero_grad(*args, **kwargs)
        self.muon.zero_grad(*args, **kwargs)

    def state_dict(self) -> dict[str, object]:
        """``{"adam": torch AdamW state, "muon": torch Muon state}``."""
        return {
            "adam": self.adamw.state_dict(),
            "muon": self.muon.state_dict(),
        }

    def load_state_dict(self, state_dict: dict[str, object]) -> None:
        """Hand each branch's entry of a :meth:`state_dict` result to its torch optimizer."""
        if "adam" in state_dict:
            self.adamw.load_state_dict(state_dict["adam"])
        if "muon" in state_dict:
            self.muon.load_state_dict(state_dict["muon"])
