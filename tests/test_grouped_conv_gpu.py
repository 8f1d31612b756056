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


class _Capture:
    """Raw captures (float64 on the CPU, fp32 on the device) and per-sample
    autograd gradients of one module."""

    def __init__(self, factory, shape, device, seed=0, module=None):
        from dattri_llm_amd.gradient import ops

        torch.manual_seed(seed)
        self.module = module if module is not None else factory().double()
        self.layer_type = f"nn.{type(self.module).__name__}"
        self.kwargs = ops.extract_module_kwargs(self.module, self.layer_type)
        self.x = torch.randn(B, *shape, dtype=torch.float64)
        out = self.module(self.x)
        self.w = torch.randn_like(out)
        self.a, self.g = self.x.float().to(device), self.w.float().to(device)
        self.ref = []
        for i in range(B):
            self.module.zero_grad()
            (self.module(self.x[i:i + 1]) * self.w[i:i + 1]).sum().backward()
            bias = self.module.bias
            self.ref.append((self.module.weight.grad.detach().clone(),
                             None if bias is None else bias.grad.detach().clone()))
        self.module.zero_grad()

    @property
    def groups(self):
        return self.module.groups

    @property
    def transposed(self):
        return "Transpose" in self.layer_type

    def ref_flat(self):
        """Per-sample gradients in the materialized layout (float64)."""
        rows = []
        for wg, bg in self.ref:
            if self.transposed:
                c_in = wg.shape[0]
                g_, c_in_g = self.groups, c_in // self.groups
                p_g = wg[0].numel()
                blocks = wg.reshape(g_, c_in_g, p_g)
                if bg is None:
                    rows.append(blocks.reshape(-1))
                    continue
                c_out_g = bg.numel() // g_
                full = torch.zeros(g_, c_in_g + 1, p_g + c_out_g, dtype=wg.dtype)
                full[:, :c_in_g, :p_g] = blocks
                full[:, -1, p_g:] = bg.reshape(g_, c_out_g)
                rows.append(full.reshape(-1))
            else:
                block = wg.reshape(wg.shape[0], -1)
                if bg is not None:
                    block = torch.cat([block, bg.unsqueeze(-1)], dim=-1)
                rows.append(block.reshape(-1))
        return torch.stack(rows)

    def pre(self):
        from dattri_llm_amd.gradient import ops

        return ops.preprocess_factors(self.a, self.g, self.layer_type, self.kwargs)


@pytest.fixture(params=_cases(), ids=[c[0] for c in _cases()])
def cap(request, device):
    _, factory, shape = request.param
    print(f"grouped conv case {request.param[0]}", flush=True)
    return _Capture(factory, shape, device)


def _second(cap_, device):
    return _Capture(None, tuple(cap_.x.shape[1:]), device, seed=1, module=cap_.module)


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
