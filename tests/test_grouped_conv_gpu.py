"""Grouped convolutions (groups > 1, depthwise included) through every op on
the MI355X kernels -- the reference's suite tests/gradient/test_grouped_conv.py
with its seven module cases, against per-sample autograd gradients of real
nn.Conv* / nn.ConvTranspose* modules in float64 on the CPU: materialization in
the parameter layout, cross / self dots and norms in every routing mode,
per-token decompositions, K-FAC factors (one covariance per group),
per-group inverses, the preconditioned Gram, the EK-FAC rotation round trip,
and the LoGRA / mask projections.  The kernels compute in fp32, so the bar
is fp32's (the reference's float64 run uses 1e-9)."""

from __future__ import annotations

import pytest
import torch
from torch import nn

pytestmark = pytest.mark.gpu

B = 3
TOL = {"rtol": 2e-5, "atol": 2e-5}


def _cases():
    return [
        ("conv1d-g2", lambda: nn.Conv1d(6, 4, 3, groups=2, padding=1), (6, 9)),
        ("conv1d-g2-nobias", lambda: nn.Conv1d(6, 4, 3, groups=2, bias=False), (6, 9)),
        ("conv1d-depthwise", lambda: nn.Conv1d(4, 4, 3, groups=4, padding=2), (4, 9)),
        ("conv2d-g2", lambda: nn.Conv2d(4, 6, (3, 2), groups=2, padding=1, stride=(1, 2)), (4, 7, 6)),
        ("conv3d-depthwise", lambda: nn.Conv3d(3, 3, 2, groups=3, padding=1), (3, 4, 4, 3)),
        ("convT1d-g2", lambda: nn.ConvTranspose1d(4, 6, 3, groups=2, padding=1), (4, 9)),
        ("convT2d-g2", lambda: nn.ConvTranspose2d(4, 4, 2, groups=2), (4, 5, 5)),
    ]


def _dense_layout(wg, bg, transposed, groups):
    """One sample's (weight, bias) gradient placed where materialize puts it.

    Convolution: a row per output channel -- its kernel weights, then its
    bias.  Transposed convolution (weight ``(C_in, C_out/g, *k)``): per group,
    a row per input channel holding its weights to the group's output
    channels, and with a bias one extra row carrying the group's output-channel
    biases past those weight columns, zero before them."""
    if not transposed:
        rows = wg.flatten(1)
        return (rows if bg is None else torch.column_stack([rows, bg])).flatten()
    per_group = wg.flatten(1).unflatten(0, (groups, -1))  # (g, C_in/g, C_out/g * prod(k))
    if bg is None:
        return per_group.flatten()
    bias = bg.unflatten(0, (groups, -1))  # (g, C_out/g)
    width = per_group.shape[-1]
    weights = nn.functional.pad(per_group, (0, bias.shape[-1]))
    bias_row = nn.functional.pad(bias, (width, 0)).unsqueeze(1)
    return torch.cat([weights, bias_row], dim=1).flatten()


class _ConvCase:
    """One module's raw captures (float64 on the host, fp32 on the device) and
    its per-sample gradients from torch.func (a vmap over samples of the
    gradient of sum(out * w))."""

    def __init__(self, module, shape, device, seed):
        from torch.func import functional_call, grad, vmap

        from dattri_llm_amd.gradient import ops

        gen = torch.Generator().manual_seed(seed)
        self.module = module
        self.layer_type = "nn." + type(module).__name__
        self.kwargs = ops.extract_module_kwargs(module, self.layer_type)
        self.x = torch.randn(B, *shape, dtype=torch.float64, generator=gen)
        with torch.no_grad():
            w = torch.randn(module(self.x).shape, dtype=torch.float64, generator=gen)
        self.a, self.g = self.x.float().to(device), w.float().to(device)
        params = {n: p.detach() for n, p in module.named_parameters()}

        def weighted_out(p, xi, wi):
            return (functional_call(module, p, (xi[None],)) * wi[None]).sum()

        per_sample = vmap(grad(weighted_out), in_dims=(None, 0, 0))(params, self.x, w)
        bias = per_sample.get("bias")
        self._flat = torch.stack([
            _dense_layout(per_sample["weight"][i], None if bias is None else bias[i], self.transposed, self.groups)
            for i in range(B)])

    @property
    def groups(self):
        return self.module.groups

    @property
    def transposed(self):
        return isinstance(self.module, nn.modules.conv._ConvTransposeNd)

    def ref_flat(self):
        """Per-sample gradients in the materialized layout (float64)."""
        return self._flat

    def pre(self):
        from dattri_llm_amd.gradient import ops

        return ops.preprocess_factors(self.a, self.g, self.layer_type, self.kwargs)


@pytest.fixture(params=_cases(), ids=[c[0] for c in _cases()])
def cap(request, device):
    _, factory, shape = request.param
    print(f"grouped conv case {request.param[0]}", flush=True)
    torch.manual_seed(0)
    return _ConvCase(factory().double(), shape, device, seed=0)


def _second(cap_, device):
    """Other samples through the same module."""
    return _ConvCase(cap_.module, tuple(cap_.x.shape[1:]), device, seed=1)


def _close(got, want, **tol):
    torch.testing.assert_close(got.double().cpu(), want.double().cpu(), **(tol or TOL))


def test_preprocess_carries_the_group_axis(cap):
    assert cap.kwargs["groups"] == cap.module.groups
    a, g = cap.pre()
    assert a.ndim == 4 and g.ndim == 4
    assert a.shape[2] == g.shape[2] == cap.groups
    assert a.shape[:3] == g.shape[:3]


def test_materialize_matches_autograd(cap):
    from dattri_llm_amd.gradient import ops

    got = ops.materialize_factors(cap.a, cap.g, cap.layer_type, cap.kwargs)
    _close(got, cap.ref_flat())
    n_params = sum(p.numel() for p in cap.module.parameters())
    if cap.transposed and cap.module.bias is not None:
        assert got.shape[1] > n_params  # the transposed bias pads each group block
    else:
        assert got.shape == (B, n_params)


@pytest.mark.parametrize("mode", ["factorized", "materialized", "auto"])
def test_cross_gram_matches_autograd(cap, device, mode):
    from dattri_llm_amd.gradient import ops

    other = _second(cap, device)
    got = ops.cross_dot_factors(cap.a, cap.g, other.a, other.g, cap.layer_type, cap.kwargs, cap.kwargs, mode=mode)
    _close(got, cap.ref_flat() @ other.ref_flat().T)


def test_self_dot_and_norms(cap):
    from dattri_llm_amd.gradient import ops

    ref = cap.ref_flat()
    _close(ops.dot_factors(cap.a, cap.g, cap.a, cap.g, cap.layer_type, cap.kwargs, cap.kwargs), (ref * ref).sum(-1))
    for mode in ("factorized", "materialized"):
        _close(ops.grad_norm_sq_factors(cap.a, cap.g, cap.layer_type, cap.kwargs, mode=mode), (ref * ref).sum(-1))


def test_per_token_decomposition_sums_to_the_gram(cap, device):
    from dattri_llm_amd.gradient import ops

    other = _second(cap, device)
    a1, g1 = cap.pre()
    a2, g2 = other.pre()
    per_token = ops.cross_gram_per_token(a1, g1, a2, g2, cap.layer_type)
    assert per_token.shape == (B, a1.shape[1], B)
    _close(per_token.sum(1), cap.ref_flat() @ other.ref_flat().T)
    dense2 = ops.materialize_factors(other.a, other.g, cap.layer_type, cap.kwargs)
    _close(ops.cross_gram_per_token_dense(a1, g1, dense2, cap.layer_type), per_token)


# -- K-FAC / EK-FAC -----------------------------------------------------------------------------


def test_kfac_factors_are_per_group_covariances(cap):
    from dattri_llm_amd.gradient import ops

    a, g = (t.double().cpu() for t in cap.pre())
    A, G = ops.kfac_factors(cap.a, cap.g, cap.layer_type, cap.kwargs)
    n_rows = a.shape[0] * a.shape[1]
    assert A.shape == (cap.groups, a.shape[-1], a.shape[-1])
    assert G.shape == (cap.groups, g.shape[-1], g.shape[-1])
    for grp in range(cap.groups):
        a_rows = a[:, :, grp].reshape(n_rows, -1)
        g_rows = g[:, :, grp].reshape(n_rows, -1)
        _close(A[grp], a_rows.T @ a_rows / n_rows)
        _close(G[grp], g_rows.T @ g_rows / n_rows)


def test_kfac_accumulator_matches_one_shot(cap, device):
    from dattri_llm_amd.gradient import ops

    other = _second(cap, device)
    acc = ops.LayerKroneckerAccumulator()
    acc.update(cap.a, cap.g, cap.layer_type, cap.kwargs)
    acc.update(other.a, other.g, cap.layer_type, cap.kwargs)
    A, G = acc.result()
    A_ref, G_ref = ops.kfac_factors(torch.cat([cap.a, other.a]), torch.cat([cap.g, other.g]), cap.layer_type,
                                    cap.kwargs)
    _close(A, A_ref, rtol=1e-5, atol=1e-6)
    _close(G, G_ref, rtol=1e-5, atol=1e-6)


def test_inverses_are_per_group(cap):
    from dattri_llm_amd.gradient import ops

    A, G = ops.kfac_factors(cap.a, cap.g, cap.layer_type, cap.kwargs)
    A_inv = ops.sym_inverse(A, 0.1)
    for grp in range(cap.groups):
        _close(A_inv[grp], ops.sym_inverse(A[grp], 0.1), rtol=1e-5, atol=1e-6)
    _close(ops.dense_inverse(G, 0.1), torch.stack([ops.dense_inverse(G[i], 0.1) for i in range(cap.groups)]),
           rtol=1e-5, atol=1e-6)


def _blocks(cap, flat):
    a, g = cap.pre()
    if cap.transposed:
        return flat.reshape(B, cap.groups, a.shape[-1], g.shape[-1])
    return flat.reshape(B, cap.groups, g.shape[-1], a.shape[-1])


def test_kfac_preconditioned_gram(cap, device):
    from dattri_llm_amd.gradient import ops

    other = _second(cap, device)
    A, G = ops.kfac_factors(cap.a, cap.g, cap.layer_type, cap.kwargs)
    A_inv, G_inv = ops.sym_inverse(A, 0.1), ops.sym_inverse(G, 0.1)
    got = ops.kfac_cross_factors(cap.a, cap.g, other.a, other.g, cap.layer_type, A_inv, G_inv, cap.kwargs,
                                 cap.kwargs)
    # the explicit per-group preconditioning of the autograd blocks (float64)
    a_i, g_i = A_inv.double().cpu(), G_inv.double().cpu()
    b1, b2 = _blocks(cap, cap.ref_flat()), _blocks(cap, other.ref_flat())
    if cap.transposed:  # blocks (C_in/G, P_g): A on the left, G on the right
        pre = torch.matmul(a_i, b1) @ g_i
    else:  # blocks (D_g, K_g): G on the left, A on the right
        pre = torch.matmul(g_i, b1) @ a_i
    ref = pre.reshape(B, -1) @ b2.reshape(B, -1).T
    _close(got, ref, rtol=1e-4, atol=1e-5)
    if not cap.transposed:
        dense1 = ops.materialize_factors(cap.a, cap.g, cap.layer_type, cap.kwargs)
        _close(ops.kfac_precondition_materialized(dense1, A_inv, G_inv), pre.reshape(B, -1), rtol=1e-4, atol=1e-5)


def test_ekfac_rotation_roundtrip(cap):
    from dattri_llm_amd.gradient import ops
    from dattri_llm_amd.gradient.ops.kronecker import _ekfac_rotate_materialized

    A, G = ops.kfac_factors(cap.a, cap.g, cap.layer_type, cap.kwargs)
    _, U_A, _, U_G = ops.kfac_eigh(A, G)
    M = ops.ekfac_materialize_factors(cap.a, cap.g, cap.layer_type, U_A, U_G, cap.kwargs)
    dense = ops.materialize_factors(cap.a, cap.g, cap.layer_type, cap.kwargs).float()
    _close(_ekfac_rotate_materialized(dense, cap.layer_type, U_A, U_G), M, rtol=1e-5, atol=1e-5)
    back = ops.ekfac_precondition(M, U_A, U_G, torch.ones_like(M[0]), cap.layer_type)
    _close(back, dense, rtol=1e-4, atol=1e-5)


# -- projections --------------------------------------------------------------------------------


def test_logra_keeps_the_group_axis(cap):
    from dattri_llm_amd.gradient import ops

    a_p, g_p = ops.project_factors(cap.a, cap.g, cap.layer_type, ops.DattriProjector(), cap.kwargs, proj_dim=4,
                                   proj_max_batch_size=8)
    a, _ = cap.pre()
    assert a_p.shape == (B, a.shape[1], cap.groups, 4)
    assert g_p.shape == (B, a.shape[1], cap.groups, 4)
    assert ops.materialize_factors(a_p, g_p, "nn.Linear").shape == (B, cap.groups * 16)


def test_mask_gathers_the_materialized_gradient(cap):
    from dattri_llm_amd.gradient import ops

    proj = ops.DattriProjector()
    full = ops.materialize_factors(cap.a, cap.g, cap.layer_type, cap.kwargs)
    k = min(12, full.shape[1])
    got = ops.mask_factors(cap.a, cap.g, cap.layer_type, proj, cap.kwargs, proj_dim=k, proj_seed=3)
    idx = proj.mask_indices(full.shape[1], proj_dim=k, proj_seed=3, device=full.device)
    _close(got, full[:, idx])
