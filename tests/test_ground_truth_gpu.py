"""Ground truth: the ops on a module's raw capture against per-sample
param.grad (the reference's tests/gradient/test_ground_truth.py).

For each supported layer family a small module runs one batched forward and
backward in fp32 on the GPU; a forward hook keeps the module's input and a
hook on its output keeps the output gradient -- the raw (a, g) a capture
records, with extract_module_kwargs.  materialize_factors, grad_norm_sq_factors
and pairwise_dot_factors on that capture are compared with the weight (and
bias) gradients of each sample run alone through a float64 copy of the module
on the CPU, in the reference's materialized layout.  The loss weights the
output by a fixed random tensor so every output gradient is non-trivial."""

from __future__ import annotations

import copy

import pytest
import torch
from torch import nn
from torch.nn.modules.linear import NonDynamicallyQuantizableLinear

pytestmark = pytest.mark.gpu

B, T, D_IN, D_OUT, VOCAB, E = 4, 5, 8, 6, 32, 10


class _QKNorm(nn.Module):
    """RMSNorm over the last axis of (B, T, heads, head_dim): the weight is
    shared across heads, so the head axis sums like the token axis."""

    def __init__(self):
        super().__init__()
        self.ln = nn.RMSNorm(4, elementwise_affine=True)

    def forward(self, x):
        b, t = x.shape[:2]
        return self.ln(x.view(b, t, 2, 4)).flatten(2)


def _flat_linear(w, b):
    m = w.reshape(w.shape[0], -1)
    return (torch.cat([m, b.unsqueeze(-1)], -1) if b is not None else m).flatten()


def _flat_hf_conv1d(w, b):  # HF Conv1D stores (I, O): the materialized layout is (O, I [+1])
    return _flat_linear(w.T, b)


def _flat_param(w, b):  # embeddings and norms: [weight | bias]
    return torch.cat([w.flatten()] + ([b.flatten()] if b is not None else []))


def _flat_conv_transpose(w, b):
    c_in, p = w.shape[0], w[0].numel()
    if b is None:
        return w.reshape(c_in, p).flatten()
    full = torch.zeros(c_in + 1, p + b.numel(), dtype=w.dtype)
    full[:c_in, :p] = w.reshape(c_in, p)
    full[-1, p:] = b
    return full.flatten()


def _ids(shape):
    return lambda gen: torch.randint(0, VOCAB, shape, generator=gen)


def _x(*shape):
    return lambda gen: torch.randn(*shape, generator=gen, dtype=torch.float64)


# (id, module factory, input maker, target attribute (None: the module itself), layer_type, flattener)
CASES = [
    ("linear-2d", lambda: nn.Linear(D_IN, D_OUT, bias=False), _x(B, D_IN), None, "nn.Linear", _flat_linear),
    ("linear-3d-bias", lambda: nn.Linear(D_IN, D_OUT), _x(B, T, D_IN), None, "nn.Linear", _flat_linear),
    ("nondynquant-bias", lambda: NonDynamicallyQuantizableLinear(D_IN, D_OUT), _x(B, T, D_IN), None,
     "nn.NonDynamicallyQuantizableLinear", _flat_linear),
    ("hf-conv1d", "hf", _x(B, T, D_IN), None, "transformers.pytorch_utils.Conv1D", _flat_hf_conv1d),
    ("embedding", lambda: nn.Embedding(VOCAB, E), _ids((B, T)), None, "nn.Embedding", _flat_param),
    ("embedding-bag-sum", lambda: nn.EmbeddingBag(VOCAB, E, mode="sum"), _ids((B, T)), None, "nn.EmbeddingBag",
     _flat_param),
    ("embedding-bag-mean", lambda: nn.EmbeddingBag(VOCAB, E, mode="mean"), _ids((B, T)), None, "nn.EmbeddingBag",
     _flat_param),
    ("layernorm", lambda: nn.LayerNorm(D_IN, bias=False), _x(B, T, D_IN), None, "nn.LayerNorm", _flat_param),
    ("layernorm-bias", lambda: nn.LayerNorm(D_IN), _x(B, T, D_IN), None, "nn.LayerNorm", _flat_param),
    ("layernorm-2d", lambda: nn.LayerNorm(D_IN), _x(B, D_IN), None, "nn.LayerNorm", _flat_param),
    ("rmsnorm", lambda: nn.RMSNorm(D_IN), _x(B, T, D_IN), None, "nn.RMSNorm", _flat_param),
    ("layernorm-width6", lambda: nn.LayerNorm(6), _x(B, T, 6), None, "nn.LayerNorm", _flat_param),
    ("rmsnorm-width5", lambda: nn.RMSNorm(5), _x(B, 5), None, "nn.RMSNorm", _flat_param),
    ("qk-norm", _QKNorm, _x(B, T, 8), "ln", "nn.RMSNorm", _flat_param),
    ("groupnorm", lambda: nn.GroupNorm(2, 4), _x(B, 4, 3, 3), None, "nn.GroupNorm", _flat_param),
    ("instancenorm2d", lambda: nn.InstanceNorm2d(4, affine=True), _x(B, 4, 3, 3), None, "nn.InstanceNorm2d",
     _flat_param),
    ("conv1d", lambda: nn.Conv1d(4, D_OUT, 3, bias=False), _x(B, 4, 7), None, "nn.Conv1d", _flat_linear),
    ("conv1d-bias", lambda: nn.Conv1d(4, D_OUT, 3), _x(B, 4, 7), None, "nn.Conv1d", _flat_linear),
    ("conv2d-bias", lambda: nn.Conv2d(3, 4, (2, 3), stride=(1, 2), padding=1), _x(B, 3, 5, 6), None, "nn.Conv2d",
     _flat_linear),
    ("conv3d", lambda: nn.Conv3d(2, 3, 2, bias=False), _x(B, 2, 3, 4, 3), None, "nn.Conv3d", _flat_linear),
    ("convT1d", lambda: nn.ConvTranspose1d(4, 3, 3, bias=False), _x(B, 4, 5), None, "nn.ConvTranspose1d",
     _flat_conv_transpose),
    ("convT1d-bias", lambda: nn.ConvTranspose1d(4, 3, 3), _x(B, 4, 5), None, "nn.ConvTranspose1d",
     _flat_conv_transpose),
    ("convT2d-bias", lambda: nn.ConvTranspose2d(3, 2, 2), _x(B, 3, 3, 4), None, "nn.ConvTranspose2d",
     _flat_conv_transpose),
    ("convT3d-bias", lambda: nn.ConvTranspose3d(2, 2, 2), _x(B, 2, 2, 3, 2), None, "nn.ConvTranspose3d",
     _flat_conv_transpose),
]


def _factory(f):
    if f == "hf":
        from transformers.pytorch_utils import Conv1D

        return Conv1D(D_OUT, D_IN)  # weight (nx, nf) = (D_IN, D_OUT)
    return f()


def _target(model, attr):
    return getattr(model, attr) if attr else model


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_ops_match_per_sample_param_grad(device, case):
    from dattri_llm_amd.gradient import ops

    name, factory, make_x, attr, lt, flatten = case
    print(f"ground truth {name}", flush=True)
    torch.manual_seed(0)
    model64 = _factory(factory).double()
    gen = torch.Generator().manual_seed(1)
    x = make_x(gen)
    w = torch.randn(model64(x).shape, generator=gen, dtype=torch.float64)

    # per-sample ground truth, float64 on the CPU
    layer64 = _target(model64, attr)
    truth = []
    for i in range(B):
        model64.zero_grad()
        (model64(x[i:i + 1]) * w[i:i + 1]).sum().backward()
        bias = getattr(layer64, "bias", None)
        truth.append(flatten(layer64.weight.grad.detach().clone(),
                             None if bias is None else bias.grad.detach().clone()))
    truth = torch.stack(truth)

    # the batched fp32 pass on the GPU, captured by hooks
    model = copy.deepcopy(model64).float().to(device)
    layer = _target(model, attr)
    cap = {}

    def keep(_mod, inputs, out):
        cap["a"] = inputs[0].detach()
        out.register_hook(lambda grad: cap.__setitem__("g", grad.detach()))

    handle = layer.register_forward_hook(keep)
    xd = x.to(device) if not x.is_floating_point() else x.float().to(device)
    (model(xd) * w.float().to(device)).sum().backward()
    handle.remove()
    mk = ops.extract_module_kwargs(layer, lt)
    a, g = cap["a"], cap["g"]

    def close(got, want, what):
        want = want.double()
        torch.testing.assert_close(got.double().cpu(), want, rtol=1e-4, atol=1e-5 * max(1.0, want.abs().max().item()),
                                   msg=lambda m: f"[{name}] {what}: {m}")

    mat = ops.materialize_factors(a, g, lt, module_kwargs=mk)
    assert mat.shape == truth.shape, (name, mat.shape, truth.shape)
    close(mat, truth, "materialize")
    close(ops.grad_norm_sq_factors(a, g, lt, mk), (truth * truth).sum(-1), "grad_norm_sq")
    close(ops.pairwise_dot_factors(a, g, lt, mk), truth @ truth.T, "pairwise_dot")
