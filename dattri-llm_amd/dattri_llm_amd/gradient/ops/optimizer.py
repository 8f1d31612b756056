"""Optimizer maps on per-sample gradients (``dattri_llm/gradient/ops/optimizer.py``).

They serve the LESS and AdamW-influence attributors, which are outside the
MI355X scoring path: the names exist so that code importing them from the ops
namespace keeps importing, and every function raises ``NotImplementedError``.
:data:`OPTIMIZER_STATE_KEYS` is the interface table of the per-parameter state
each ``torch.optim`` optimizer keeps (``state[param][key]``), as
optimizer.py:32-43 lists it.
"""

from __future__ import annotations

OPTIMIZER_STATE_KEYS: dict[str, tuple[str, ...]] = {
    "SGD": ("momentum_buffer",),
    "Adam": ("exp_avg", "exp_avg_sq", "max_exp_avg_sq"),
    "AdamW": ("exp_avg", "exp_avg_sq", "max_exp_avg_sq"),
    "Adamax": ("exp_avg", "exp_inf"),
    "NAdam": ("exp_avg", "exp_avg_sq", "mu_product"),
    "RAdam": ("exp_avg", "exp_avg_sq"),
    "RMSprop": ("square_avg", "grad_avg", "momentum_buffer"),
    "Adagrad": ("sum",),
    "Adadelta": ("square_avg", "acc_delta"),
    "Lion": ("exp_avg",),
}


def _outside(name: str):
    def fn(*_args, **_kwargs):
        raise NotImplementedError(
            f"{name} belongs to the optimizer-aware attributors (LESS, AdamW-influence), which are outside "
            "the MI355X scoring path."
        )

    fn.__name__ = name
    fn.__doc__ = f"``{name}`` (dattri_llm/gradient/ops/optimizer.py): not on the MI355X scoring path; raises."
    return fn


precondition = _outside("precondition")
adam_preconditioner = _outside("adam_preconditioner")
adamw_influence_push = _outside("adamw_influence_push")
adamw_influence_transition = _outside("adamw_influence_transition")
adamw_influence_coupling = _outside("adamw_influence_coupling")

__all__ = [
    "OPTIMIZER_STATE_KEYS",
    "adam_preconditioner",
    "adamw_influence_coupling",
    "adamw_influence_push",
    "adamw_influence_transition",
    "precondition",
]
