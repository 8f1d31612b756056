"""Gradient capture fused into autograd for ``nn.Linear`` layers.

The reference captures a linear layer's factors with a forward hook (stashing
the input activation on a per-device stack) and a backward hook that pops it,
projects both factors and either keeps them or contracts them into the
per-sample ``(B, k_g * k_a)`` block (``gradient/hooks/hooks.py:552-688``);
its ``invasive_linear_io`` variant also routes the forward through an autograd
function whose backward skips the ``d_out x d_in`` weight-gradient product the
capture never reads (``gradient/hooks/override_layers/invasive_linear.py:35-77``).

Here the capture *is* the layer's backward.  :class:`FusedCapture` routes each
selected layer's forward through :class:`_CaptureLinear`, which saves the input
(what ``nn.Linear`` saves anyway) and, in backward, returns the input gradient
and runs the capture on ``(input, grad_output)`` on the same stream:

* projected, materialized: one ``da_project_outer`` launch reads the input and
  the output gradient once and writes the ``(B, k_g * k_a)`` block (projection,
  bias row and per-sample outer-product sum fused; no ``a_p`` / ``g_p`` in HBM);
* projected, factorized: the two projected factors (``da_project_rows``);
* unprojected: the raw factors, or the dense ``(B, d_out * (d_in + 1))``
  gradient from the dW kernel.

No weight or bias gradient is produced for a captured layer, as with the
reference's invasive capture: use it for attribution, not for training.  The
representation of a layer is fixed by its first micro-batch of a step, and
the capture-style rule (``should_materialize``) decides it, as in the reference.
"""

from __future__ import annotations

import threading

import torch
from torch import nn

from dattri_llm_amd.gradient.gradient import Factorized, Gradient
from dattri_llm_amd.gradient.ops import materialize_factors, project_layer, should_materialize
from dattri_llm_amd.gradient.ops.projection import DattriProjector


class _CaptureLinear(torch.autograd.Function):
    """``F.linear`` whose backward captures the layer instead of forming its
    weight gradient (the input gradient is unchanged)."""

    @staticmethod
    def forward(ctx, x, weight, bias, slot):
        ctx.save_for_backward(x, weight)
        ctx.slot = slot
        return nn.functional.linear(x, weight, bias)

    @staticmethod
    def backward(ctx, grad_out):
        x, weight = ctx.saved_tensors
        grad_in = grad_out @ weight.to(grad_out.dtype) if ctx.needs_input_grad[0] else None
        ctx.slot.capture(x, grad_out)
        return grad_in, None, None, None


class _LayerSlot:
    """One captured layer: its settings and the parts of the current step."""

    def __init__(self, name: str, module: nn.Linear, session: FusedCapture) -> None:
        self.name, self.module, self.session = name, module, session
        self.parts: list = []
        self.factorized: bool | None = None
        self.lock = threading.Lock()

    def capture(self, x: torch.Tensor, g: torch.Tensor) -> None:
        s = self.session
        if not s.batch_first:
            x, g = x.transpose(0, 1), g.transpose(0, 1)
        mk = {"has_bias": self.module.bias is not None}
        if x.ndim == 2:
            x, g = x.unsqueeze(1), g.unsqueeze(1)
        x, g = x.detach(), g.detach()
        if s.proj_dim is None:
            seq_len = x.shape[1]
            keep = self.factorized
            if keep is None:
                keep = not should_materialize(s.capture_style, seq_len, x.shape[-1] + 1, g.shape[-1])
            part = (x, g) if keep else materialize_factors(x, g, "nn.Linear", mk, s.include_bias)
        else:
            style = s.capture_style
            if self.factorized is not None:  # a step never mixes the two representations
                style = "factorized" if self.factorized else "materialized"
            part, keep = project_layer(
                Factorized(x, g, module_kwargs=mk), "nn.Linear", s.projector, style="logra",
                capture_style=style, proj_dim=s.proj_dim, proj_seed=s.proj_seed,
                include_bias=s.include_bias,
            )
        with self.lock:
            self.factorized = keep
            self.parts.append(part)

    def collect(self):
        with self.lock:
            parts, keep = list(self.parts), self.factorized
        if not parts:
            return None
        if keep:
            a = torch.cat([p[0] for p in parts], dim=0)
            g = torch.cat([p[1] for p in parts], dim=0)
            mk = {"has_bias": self.module.bias is not None} if self.session.proj_dim is None else None
            return "factorized", Factorized(a, g, module_kwargs=mk)
        return "materialized", torch.cat(parts, dim=0)

    def clear(self) -> None:
        with self.lock:
            self.parts.clear()
            self.factorized = None


class FusedCapture:
    """Capture per-sample gradients of ``nn.Linear`` layers inside autograd.

    ``layers``: names of the ``nn.Linear`` modules to capture (default: all).
    ``proj_dim``: LoGRA projection width (``None``: unprojected capture), with
    ``proj_seed`` / ``projector`` as in ``project_factors`` (seed for the
    gradient side, seed + 1 for the activation side).  ``capture_style``:
    ``"factorized"``, ``"materialized"`` or ``"auto"`` (``should_materialize``).

    Use as a context manager around forward + backward passes; each backward
    appends one micro-batch per layer.  :meth:`gradient` returns the captured
    block as a :class:`Gradient` (``RuntimeError`` when nothing was captured),
    :meth:`clear` starts the next step.  Each
    captured layer must run once per forward."""

    def __init__(self, model: nn.Module, layers=None, *, proj_dim: int | None = None, proj_seed: int = 0,
                 projector=None, capture_style: str = "factorized", batch_first: bool = True,
                 include_bias: bool = True) -> None:
        if capture_style not in ("factorized", "materialized", "auto"):
            raise ValueError(f"capture_style must be 'factorized', 'materialized' or 'auto', got {capture_style!r}.")
        root = getattr(model, "module", model)
        wanted = None if layers is None else set(layers)
        self.slots: dict[str, _LayerSlot] = {}
        for name, module in root.named_modules():
            if wanted is not None and name not in wanted:
                continue
            if type(module) is not nn.Linear:
                if wanted is not None:
                    raise ValueError(f"layer {name!r} is a {type(module).__name__}, not a plain nn.Linear")
                continue
            self.slots[name] = _LayerSlot(name, module, self)
        if wanted is not None and wanted - set(self.slots):
            raise ValueError(f"no such layers: {sorted(wanted - set(self.slots))}")
        self.proj_dim, self.proj_seed = proj_dim, proj_seed
        self.projector = DattriProjector.coerce(projector)
        self.capture_style, self.batch_first, self.include_bias = capture_style, batch_first, include_bias
        self._reverts: list = []

    def __enter__(self) -> FusedCapture:
        for slot in self.slots.values():
            m = slot.module

            def forward(x, _m=m, _slot=slot):
                return _CaptureLinear.apply(x, _m.weight, _m.bias, _slot)

            had = "forward" in m.__dict__
            old = m.__dict__.get("forward")
            m.forward = forward
            self._reverts.append((m, had, old))
        return self

    def __exit__(self, *_exc) -> bool:
        while self._reverts:
            m, had, old = self._reverts.pop()
            if had:
                m.forward = old
            else:
                del m.forward
        return False

    def gradient(self) -> Gradient:
        rep, data, types = {}, {}, {}
        for name, slot in self.slots.items():
            got = slot.collect()
            if got is None:
                continue
            rep[name], data[name] = got
            types[name] = "nn.Linear"
        if not data:
            raise RuntimeError("FusedCapture: no layer has been captured since the last clear()")
        return Gradient(rep, data, types)

    def clear(self) -> None:
        for slot in self.slots.values():
            slot.clear()


__all__ = ["FusedCapture"]
