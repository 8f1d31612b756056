"""Random projection of per-sample gradients on the MI355X kernels.

Mirrors ``dattri_llm/gradient/ops/projection.py`` for the ``"logra"`` style:

* :class:`DattriProjector` (projection.py:93-328) builds a layer's ``(d, k)``
  matrix once from a projector factory following dattri's ``random_project``
  protocol -- ``factory(feature, batch_size, *, proj_dim, proj_seed, device,
  **kw) -> callable(x)`` -- by projecting identity chunks through it, and
  caches it.  dattri itself is not available here, so the default factory is
  :func:`gaussian_projector`, this package's own seeded Gaussian map (its
  values are not dattri's; any dattri-protocol factory can be passed instead).
* :class:`ProjectionMatrix` (projection.py:331-370) applies it with the
  ``da_project_rows`` kernel; the bias row of a linear layer is a broadcast
  add, so the ones-augmented activation is never formed.
* the activation side uses ``proj_seed + 1`` and the gradient side
  ``proj_seed`` (projection.py:437-440, :476-488).
* when the capture style materializes the projected factors
  (:func:`should_materialize`, projection.py:846-899), the projection of both
  factors and the per-sample outer-product sum run as ONE kernel
  (``da_project_outer``) that reads each factor row once.

The other two styles of ``project_layer`` (projection.py:902-944):

* ``"dense"`` (TRAK): the per-sample gradient from the dW kernel, then one
  row projection (:func:`project_materialized_factors`, projection.py:396-420);
* ``"mask"``: ``proj_dim`` fixed random coordinates of the per-sample gradient
  (:func:`mask_factors`, projection.py:687-811), gathered from the factors by
  the ``da_gather_entries`` kernel without forming the gradient; the subset is
  drawn as the reference draws it (a CPU generator seeded from ``(proj_seed,
  width, proj_dim)``), so masked captures interchange.

Layer families (projection.py:440-489, :718-775): linear layers, convolutions
(the unfolded factors, a grouped one per group with shared matrices; masks in
the per-group (rows, columns) layout, transposed for ConvTranspose) and
embeddings (the input-side projection of a token is a row of the
``(num_embeddings, proj_dim)`` matrix; a mask entry (v, e) sums the gradient
column e over the tokens with id v, ``da_gather_embedding_entries``).
"""

from __future__ import annotations

import math

import torch

from dattri_llm_amd import kernels
from dattri_llm_amd.gradient.ops import conv, dtypes
from dattri_llm_amd.gradient.ops import embedding as emb
from dattri_llm_amd.gradient.ops.materialize import linear_dense, materialize_factors
from dattri_llm_amd.gradient.ops.preprocess import final_linear, preprocess_factors, to_3d
from dattri_llm_amd.gradient.ops.types import (
    is_conv,
    is_conv_transpose,
    is_embedding,
    is_linear,
    is_norm,
    require_supported,
)
from dattri_llm_amd.utils.cache import TensorCache

PROJECTION_STYLES = ("logra", "dense", "mask")
CAPTURE_STYLES = ("factorized", "materialized", "auto")
MASK_KEYS = frozenset({"style", "proj_dim", "proj_seed", "include_bias", "device"})
_IDENTITY_CHUNK_ROWS = 8192
_FUSED_MAX_WIDTH = 64


def mask_seed(proj_seed: int, d: int, proj_dim: int) -> int:
    """Generator seed of a ``"mask"`` coordinate subset, one per ``(seed, width,
    size)`` -- the reference's formula (projection.py:78-80), so masked
    gradients from both implementations keep the same coordinates."""
    return ((proj_seed * 1_000_003 + d) * 1_000_003 + proj_dim) & ((1 << 63) - 1)


def gaussian_matrix(d: int, proj_dim: int, proj_seed: int) -> torch.Tensor:
    """The default projector's ``(d, proj_dim)`` float32 matrix: i.i.d.
    N(0, 1/proj_dim) entries drawn on the CPU from ``proj_seed``, so every
    device and process gets the same map."""
    gen = torch.Generator(device="cpu").manual_seed(int(proj_seed))
    return torch.randn(d, proj_dim, generator=gen, dtype=torch.float32) / math.sqrt(proj_dim)


def gaussian_projector(feature, batch_size, *, proj_dim: int, proj_seed: int = 0, device=None, **_kw):
    """A dattri-protocol projector factory over :func:`gaussian_matrix`."""
    d = feature.shape[-1]
    matrix = gaussian_matrix(d, proj_dim, proj_seed)
    dev = torch.device(device) if device is not None else feature.device
    matrix = matrix.to(dev)

    def project(x, ensemble_id=0):  # noqa: ARG001 - protocol
        return x.to(matrix.dtype) @ matrix

    project.matrix = matrix
    return project


def _projector_key(projector) -> str:
    return f"{getattr(projector, '__module__', '')}.{getattr(projector, '__qualname__', repr(projector))}"


class DattriProjector:
    """A projection factory plus the cache of the matrices it builds."""

    def __init__(self, projector=None, *, cache: TensorCache | None = None) -> None:
        self._factory = projector
        self._cache = cache if cache is not None else TensorCache("memory")

    @classmethod
    def coerce(cls, projector):
        return projector if isinstance(projector, DattriProjector) else cls(projector)

    @property
    def factory(self):
        if self._factory is None:
            self._factory = gaussian_projector
        return self._factory

    @property
    def cache(self) -> TensorCache:
        return self._cache

    def matrix(self, d_in: int, *, proj_dim: int, proj_seed: int, device, dtype, **proj_kwargs) -> torch.Tensor:
        """The ``(d_in, proj_dim)`` matrix the factory applies, built once
        (projection.py:150-200): identity chunks pushed through the factory."""
        key = (_projector_key(self.factory), d_in, proj_dim, proj_seed, str(device), dtype,
               tuple(sorted((k, repr(v)) for k, v in proj_kwargs.items())))
        cached = self._cache.get(key)
        if cached is not None:
            return cached
        if self.factory is gaussian_projector:
            matrix = gaussian_matrix(d_in, proj_dim, proj_seed).to(device=device, dtype=dtype)
        else:
            rows = []
            for start in range(0, d_in, _IDENTITY_CHUNK_ROWS):
                stop = min(start + _IDENTITY_CHUNK_ROWS, d_in)
                block = torch.zeros(stop - start, d_in, device=device, dtype=torch.float32)
                idx = torch.arange(stop - start, device=device)
                block[idx, idx + start] = 1.0
                fn = self.factory(block, block.shape[0], proj_dim=proj_dim, proj_seed=proj_seed,
                                  device=device, **proj_kwargs)
                rows.append(fn(block))
            matrix = torch.cat(rows, dim=0).to(dtype)
        self._cache.put(key, matrix)
        return matrix

    def apply(self, x: torch.Tensor, *, proj_dim: int, proj_seed: int = 0, include_bias: bool = False,
              **proj_kwargs) -> torch.Tensor:
        """Project the last axis of *x* to ``proj_dim`` (projection.py:235-280)."""
        (x,) = dtypes.as_float(x)
        device = torch.device(proj_kwargs.pop("device", x.device))
        x = x.to(device)
        pm = self.resolve(x.shape[-1], proj_dim=proj_dim, proj_seed=proj_seed, include_bias=include_bias,
                          device=device, dtype=x.dtype, **proj_kwargs)
        return pm(x)

    def resolve(self, d_in: int, *, proj_dim: int, proj_seed: int = 0, include_bias: bool = False,
                device, dtype, **proj_kwargs) -> ProjectionMatrix:
        """The projection :meth:`apply` would perform, resolved once (projection.py:282-311)."""
        device = torch.device(proj_kwargs.pop("device", device))
        matrix = self.matrix(d_in + (1 if include_bias else 0), proj_dim=proj_dim, proj_seed=proj_seed,
                             device=device, dtype=dtype, **proj_kwargs)
        return ProjectionMatrix(matrix, include_bias, d_in, dtype, device)

    def mask_indices(self, d: int, *, proj_dim: int, proj_seed: int, device) -> torch.Tensor:
        """The sorted ``(proj_dim,)`` coordinates of a width-``d`` flat gradient
        that a ``"mask"`` capture keeps (projection.py:202-233): drawn without
        replacement on the CPU from :func:`mask_seed`, so every device and
        process keeps the same subset.  Cached with the matrices."""
        if not 0 < proj_dim <= d:
            raise ValueError(f"a mask needs 0 < proj_dim <= d, got proj_dim={proj_dim} for a width-{d} layer.")
        key = ("subset", d, proj_dim, proj_seed, str(device))
        cached = self._cache.get(key)
        if cached is None:
            gen = torch.Generator(device="cpu").manual_seed(mask_seed(proj_seed, d, proj_dim))
            cached = torch.randperm(d, generator=gen)[:proj_dim].sort().values.to(device)
            self._cache.put(key, cached)
        return cached

    def clear(self) -> None:
        self._cache.clear()

    def close(self) -> None:
        self._cache.clear()

    def __enter__(self):
        return self

    def __exit__(self, *_exc) -> bool:
        self.close()
        return False


class ProjectionMatrix:
    """One layer's projection with everything but the kernel done
    (projection.py:331-370).  Holds the transposed matrix the kernel reads and
    the bias row in fp32."""

    __slots__ = ("_bias32", "_pt", "bias_row", "d_in", "device", "dtype", "matrix", "proj_dim")

    def __init__(self, matrix: torch.Tensor, include_bias: bool, d_in: int, dtype, device) -> None:
        self.matrix = matrix[:-1] if include_bias else matrix
        self.bias_row = matrix[-1] if include_bias else None
        self.d_in, self.dtype, self.device = d_in, dtype, torch.device(device)
        self.proj_dim = matrix.shape[1]
        kd = dtypes.kernel_dtype(dtype)
        self._pt = self.matrix.t().to(kd).contiguous()
        self._bias32 = self.bias_row.to(torch.float32).contiguous() if self.bias_row is not None else None

    def matches(self, x: torch.Tensor) -> bool:
        return x.shape[-1] == self.d_in and x.dtype == self.dtype and x.device == self.device

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        """Project the last axis of *x* (``(..., d_in)`` to ``(..., proj_dim)``)."""
        if x.shape[-1] != self.d_in:
            raise ValueError(f"projection expects width {self.d_in}, got {x.shape[-1]}")
        kd = dtypes.kernel_dtype(self.dtype)
        out = kernels.project_rows(x.to(kd), self._pt, bias=self._bias32, out_dtype=kd)
        return out.to(self.dtype)

    @property
    def transposed(self) -> torch.Tensor:
        """The (proj_dim, d_in) operand the kernels read."""
        return self._pt

    @property
    def bias32(self):
        return self._bias32


def apply_projection(projector, x: torch.Tensor, *, proj_dim: int, proj_seed: int = 0,
                     include_bias: bool = False, **proj_kwargs) -> torch.Tensor:
    """:meth:`DattriProjector.apply` for a factory or a projector (projection.py:373-393)."""
    return DattriProjector.coerce(projector).apply(x, proj_dim=proj_dim, proj_seed=proj_seed,
                                                   include_bias=include_bias, **proj_kwargs)


def _linear_only(layer_type: str, what: str) -> None:
    if is_norm(layer_type):
        raise ValueError(
            f"factorized projection is undefined for {layer_type!r}: its gradient is not an outer "
            "product of the factors -- use materialized projection"
        )
    if not (is_linear(layer_type) or is_embedding(layer_type) or is_conv(layer_type)
            or is_conv_transpose(layer_type)):
        require_supported(layer_type, what)


def _embedding_vocab(module_kwargs, what: str) -> int:
    if module_kwargs is None:
        raise ValueError(
            f"{what} of an embedding requires module_kwargs with 'num_embeddings' (the one-hot width "
            "cannot be inferred from the captured factors)."
        )
    return int(module_kwargs["num_embeddings"])


def _outer_sides(a, g, layer_type, projector, module_kwargs, include_bias, proj_dim, proj_seed, proj_kwargs):
    """Projected ``(a_p, g_p)`` of an embedding or convolution (projection.py:457-489).

    Embedding: a linear layer over one-hot ids, so the input-side projection of
    token v is row v of the ``(num_embeddings, proj_dim)`` matrix -- gathered
    instead of multiplying a one-hot tensor (the same values: one 1.0 times each
    entry).  The one-hot is integer, so that side resolves its dtype alone
    (fp32 under "auto"), as the reference's one-hot projection does.
    Convolution: the unfolded factors (a grouped one keeps its group axis and
    every group uses the same matrices), the conv bias an implicit ones column
    (the matrix's last row)."""
    if is_embedding(layer_type):
        vocab = _embedding_vocab(module_kwargs, "Factorized projection")
        ids, g = preprocess_factors(a, g, layer_type, module_kwargs, include_bias)
        emb.check_ids(ids, vocab=vocab)
        (g_f,) = dtypes.align(to_3d(g))
        g_p = apply_projection(projector, g_f, proj_dim=proj_dim, proj_seed=proj_seed, **proj_kwargs)
        kw = dict(proj_kwargs)
        device = torch.device(kw.pop("device", g_f.device))
        m = DattriProjector.coerce(projector).matrix(vocab, proj_dim=proj_dim, proj_seed=proj_seed + 1,
                                                     device=device, dtype=dtypes.resolve(ids), **kw)
        return m[ids.to(device)], g_p
    c = conv.final(a, g, layer_type, module_kwargs, include_bias)
    x, y = dtypes.align(c.a, c.g)
    p_in, p_out = _resolve_pair(projector, x, y, c.bias, proj_dim, proj_seed, proj_kwargs)
    return p_in(x.to(p_in.device)), p_out(y.to(p_out.device))


def _resolve_pair(projector, a, g, bias, proj_dim, proj_seed, proj_kwargs):
    proj = DattriProjector.coerce(projector)
    kw = dict(proj_kwargs)
    device = torch.device(kw.pop("device", g.device))
    dtype = dtypes.resolve(a, g)
    p_in = proj.resolve(a.shape[-1], proj_dim=proj_dim, proj_seed=proj_seed + 1, include_bias=bias,
                        device=device, dtype=dtype, **kw)
    p_out = proj.resolve(g.shape[-1], proj_dim=proj_dim, proj_seed=proj_seed, device=device,
                         dtype=dtype, **kw)
    return p_in, p_out


def project_factors(a, g, layer_type: str, projector, module_kwargs: dict | None = None,
                    include_bias: bool = True, *, proj_dim: int, proj_seed: int = 0, **proj_kwargs):
    """LoGRA: project both factors, keeping the outer-product structure
    (projection.py:423-489).  Returns ``(a_p, g_p)``."""
    _linear_only(layer_type, "project_factors")
    if not is_linear(layer_type):
        return _outer_sides(a, g, layer_type, projector, module_kwargs, include_bias, proj_dim, proj_seed,
                            proj_kwargs)
    bias = bool(module_kwargs is not None and module_kwargs["has_bias"] and include_bias)
    a, g = dtypes.align(to_3d(a), to_3d(g))
    p_in, p_out = _resolve_pair(projector, a, g, bias, proj_dim, proj_seed, proj_kwargs)
    return p_in(a.to(p_in.device)), p_out(g.to(p_out.device))


def project_activation(a, layer_type: str, projector, module_kwargs: dict | None, include_bias: bool = True,
                       *, proj_dim: int, proj_seed: int = 0, **proj_kwargs) -> torch.Tensor:
    """Project only a linear layer's activation (forward hook, projection.py:492-529)."""
    if not is_linear(layer_type):
        raise ValueError(f"project_activation is for linear layers only, got {layer_type!r}.")
    with_bias = module_kwargs is not None and module_kwargs["has_bias"] and include_bias
    a_f = to_3d(dtypes.align(a)[0])
    return apply_projection(projector, a_f, proj_dim=proj_dim, proj_seed=proj_seed + 1,
                            include_bias=with_bias, **proj_kwargs)


def project_gradient(g, layer_type: str, projector, module_kwargs: dict | None, *, proj_dim: int,
                     proj_seed: int = 0, **proj_kwargs) -> torch.Tensor:
    """Project only a linear layer's gradient (backward hook, projection.py:532-560)."""
    if not is_linear(layer_type):
        raise ValueError(f"project_gradient is for linear layers only, got {layer_type!r}.")
    g_f = to_3d(dtypes.align(g)[0])
    return apply_projection(projector, g_f, proj_dim=proj_dim, proj_seed=proj_seed, **proj_kwargs)


def project_outer_factors(a, g, layer_type: str, projector, module_kwargs: dict | None = None,
                          include_bias: bool = True, *, proj_dim: int, proj_seed: int = 0,
                          **proj_kwargs) -> torch.Tensor:
    """``materialize_factors(*project_factors(...), "nn.Linear")`` in one pass:
    the fused projection + per-sample outer-product kernel.  Returns
    ``(B, k_g * k_a)``, index ``o * k_a + i``."""
    _linear_only(layer_type, "project_outer_factors")
    if not is_linear(layer_type):  # the projected pair, then the dW kernel ("nn.Linear" layout, per group)
        a_p, g_p = _outer_sides(a, g, layer_type, projector, module_kwargs, include_bias, proj_dim, proj_seed,
                                proj_kwargs)
        return materialize_factors(a_p, g_p, "nn.Linear")
    bias = bool(module_kwargs is not None and module_kwargs["has_bias"] and include_bias)
    a, g = dtypes.align(to_3d(a), to_3d(g))
    p_in, p_out = _resolve_pair(projector, a, g, bias, proj_dim, proj_seed, proj_kwargs)
    return fused_outer(a, g, p_in, p_out)


def fused_outer(a, g, p_in: ProjectionMatrix, p_out: ProjectionMatrix) -> torch.Tensor:
    """(B, kg*ka) outer-product sum of the two projections of raw factors."""
    out_dtype = dtypes.resolve(a, g)
    kd = dtypes.kernel_dtype(out_dtype)
    if p_in.proj_dim <= _FUSED_MAX_WIDTH and p_out.proj_dim <= _FUSED_MAX_WIDTH:
        out = kernels.project_outer(a.to(kd), g.to(kd), p_in.transposed, p_out.transposed,
                                    bias_in=p_in.bias32, out_dtype=kd)
        return out.to(out_dtype)
    # wider projections: the two row projections, then the dW kernel
    return linear_dense(p_in(a), p_out(g), False).to(out_dtype)


def capture_projected(a_p: torch.Tensor, g: torch.Tensor, p_out: ProjectionMatrix, materialize: bool):
    """Backward-hook step of the LoGRA capture (hooks.py:631-648): the activation
    was projected in the forward hook; project the gradient and either keep
    the factor pair or contract it into the ``(B, k_g * k_a)`` per-sample block.
    The contraction reads ``g`` once (identity projection on the small a_p side)."""
    a_p, g = to_3d(a_p), to_3d(g)
    if not materialize:
        return a_p, p_out(g)
    ka = a_p.shape[-1]
    ident = ProjectionMatrix(torch.eye(ka, dtype=p_out.dtype, device=p_out.device), False, ka,
                             p_out.dtype, p_out.device)
    return fused_outer(a_p.to(p_out.dtype), g.to(p_out.dtype), ident, p_out)


def project_materialized_factors(a, g, layer_type: str, projector, module_kwargs: dict | None = None,
                                 include_bias: bool = True, *, proj_dim: int, proj_seed: int = 0,
                                 **proj_kwargs) -> torch.Tensor:
    """TRAK style (projection.py:396-420): the per-sample gradient (dW or norm
    kernel), then one projection of it to ``(B, proj_dim)``."""
    dense = materialize_factors(a, g, layer_type, module_kwargs, include_bias)
    return apply_projection(projector, dense, proj_dim=proj_dim, proj_seed=proj_seed, **proj_kwargs)


def project_materialized(f, layer_type: str, projector, *, proj_dim: int, include_bias: bool = True,
                         proj_seed: int = 0, **proj_kwargs) -> torch.Tensor:
    """:func:`project_materialized_factors` on a :class:`Factorized`, or the
    projection of an already dense ``(B, D)`` block (projection.py:563-596)."""
    if isinstance(f, torch.Tensor):
        return apply_projection(projector, f.reshape(f.shape[0], -1), proj_dim=proj_dim, proj_seed=proj_seed,
                                **proj_kwargs)
    bf = f.as_batch_first()
    return project_materialized_factors(bf.activation, bf.pre_activation_grad, layer_type, projector,
                                        bf.module_kwargs, include_bias, proj_dim=proj_dim, proj_seed=proj_seed,
                                        **proj_kwargs)


def _mask_options(proj_kwargs: dict, default_device) -> torch.device:
    unknown = set(proj_kwargs) - MASK_KEYS
    if unknown:
        raise ValueError(
            "style 'mask' keeps coordinates rather than projecting, so it takes only "
            f"{sorted(MASK_KEYS - {'style'})}; got unexpected {sorted(unknown)}."
        )
    return torch.device(proj_kwargs.get("device", default_device))


def mask_coordinates(projection: dict | None, layer_name: str, width: int, projector,
                     device="cpu") -> torch.Tensor | None:
    """The coordinates a ``"mask"`` capture of ``layer_name`` kept
    (projection.py:628-659), from the capture's projection config; None when
    the layer is not masked.  Any other style raises: a projected gradient's
    entries are not coordinates."""
    if projection is None:
        return None
    kw = projection.get(layer_name, projection.get("__default__"))
    if kw is None:
        return None
    style = kw.get("style", "logra")
    if style != "mask":
        raise ValueError(
            f"layer {layer_name!r} is captured with style {style!r}; coordinate-wise maps need exact gradient "
            "entries, i.e. no projection or style 'mask'."
        )
    return DattriProjector.coerce(projector).mask_indices(width, proj_dim=kw["proj_dim"],
                                                          proj_seed=kw.get("proj_seed", 0), device=torch.device(device))


def mask_materialized(x: torch.Tensor, projector, *, proj_dim: int, proj_seed: int = 0,
                      **proj_kwargs) -> torch.Tensor:
    """``proj_dim`` fixed random coordinates of a dense ``(..., D)`` block
    (projection.py:662-684)."""
    device = _mask_options(proj_kwargs, x.device)
    x = x.to(device)
    idx = DattriProjector.coerce(projector).mask_indices(x.shape[-1], proj_dim=proj_dim, proj_seed=proj_seed,
                                                         device=device)
    return x.index_select(-1, idx)


def mask_factors(a, g, layer_type: str, projector, module_kwargs: dict | None = None, include_bias: bool = True,
                 *, proj_dim: int, proj_seed: int = 0, **proj_kwargs) -> torch.Tensor:
    """``materialize_factors(...)[:, mask]`` without materializing
    (projection.py:687-783): linear layers gather each kept entry
    ``sum_t g[b,t,o] * a[b,t,i]`` straight from the factors (``da_gather_entries``,
    flat index ``o*(K+bias) + i``); norm layers are small and are materialized
    (norm kernel), then gathered.  Returns ``(B, proj_dim)``."""
    device = _mask_options(proj_kwargs, g.device)
    proj = DattriProjector.coerce(projector)
    if is_norm(layer_type):
        dense = materialize_factors(a, g, layer_type, module_kwargs, include_bias).to(device)
        idx = proj.mask_indices(dense.shape[-1], proj_dim=proj_dim, proj_seed=proj_seed, device=device)
        return dense.index_select(-1, idx)
    if is_embedding(layer_type):  # entry (v, e): the gradient column e summed over the tokens with id v
        vocab = _embedding_vocab(module_kwargs, "Subsetting")
        ids, rows_g = emb.side(a, g, layer_type, module_kwargs)
        emb.check_ids(a, vocab=vocab)
        (rows_g,) = dtypes.align(rows_g)
        out_dtype = rows_g.dtype
        e = rows_g.shape[-1]
        idx = proj.mask_indices(vocab * e, proj_dim=proj_dim, proj_seed=proj_seed, device=device)
        got = kernels.gather_embedding_entries(ids.to(device), rows_g.to(device=device,
                                               dtype=dtypes.kernel_dtype(out_dtype)), idx // e, idx % e)
        return got.to(out_dtype)
    if is_conv(layer_type) or is_conv_transpose(layer_type) or (module_kwargs is None and to_3d(a).ndim == 4):
        return _mask_conv(a, g, layer_type, proj, module_kwargs, include_bias, proj_dim, proj_seed, device)
    if not is_linear(layer_type):
        require_supported(layer_type, "mask_factors")
    x, y, bias = final_linear(a, g, layer_type, module_kwargs, include_bias)
    out_dtype = dtypes.resolve(x, y)
    x, y = (t.to(device=device, dtype=dtypes.kernel_dtype(out_dtype)) for t in dtypes.align(to_3d(x), to_3d(y)))
    if x.ndim == 4:
        raise NotImplementedError("grouped (4-D) factors are conv-only and outside this path")
    cols = x.shape[-1] + int(bias)
    idx = proj.mask_indices(y.shape[-1] * cols, proj_dim=proj_dim, proj_seed=proj_seed, device=device)
    return kernels.gather_entries(x, y, idx // cols, idx % cols, bias=bias).to(out_dtype)


def _mask_conv(a, g, layer_type, proj, module_kwargs, include_bias, proj_dim, proj_seed, device):
    """Kept entries of a convolution's gradient in materialize's layout
    (projection.py:737-775): ``o * K + i`` (conv), ``c * P + p`` (transposed),
    per group for grouped factors -- whose groups fold into the feature axes,
    so an entry's row and column come from the same group."""
    c = conv.final(a, g, layer_type, module_kwargs, include_bias)
    x, y = c.a, c.g
    if c.bias:  # an explicit ones column keeps the per-group index arithmetic plain
        x = torch.cat([x, torch.ones_like(x[..., :1])], dim=-1)
    out_dtype = dtypes.resolve(x, y)
    x, y = (t.to(device=device, dtype=dtypes.kernel_dtype(out_dtype)) for t in dtypes.align(x, y))
    groups = c.groups if x.dim() == 4 else 1
    wa, wg = x.shape[-1], y.shape[-1]
    if x.dim() == 4:
        x, y = x.reshape(*x.shape[:2], groups * wa), y.reshape(*y.shape[:2], groups * wg)
    idx = proj.mask_indices(groups * wa * wg, proj_dim=proj_dim, proj_seed=proj_seed, device=device)
    grp, rem = idx // (wa * wg), idx % (wa * wg)
    if c.transpose:  # blocks (Wa, Wg): rows from a, columns from g
        got = kernels.gather_entries(y, x, grp * wa + rem // wg, grp * wg + rem % wg)
    else:  # blocks (Wg, Wa): rows from g, columns from a
        got = kernels.gather_entries(x, y, grp * wg + rem // wa, grp * wa + rem % wa)
    return got.to(out_dtype)


def mask_factorized(f, layer_type: str, projector, *, proj_dim: int, include_bias: bool = True,
                    proj_seed: int = 0, **proj_kwargs) -> torch.Tensor:
    """:func:`mask_factors` on a :class:`Factorized`, or
    :func:`mask_materialized` of a dense ``(B, D)`` block (projection.py:814-843)."""
    if isinstance(f, torch.Tensor):
        return mask_materialized(f.reshape(f.shape[0], -1), projector, proj_dim=proj_dim, proj_seed=proj_seed,
                                 **proj_kwargs)
    bf = f.as_batch_first()
    return mask_factors(bf.activation, bf.pre_activation_grad, layer_type, projector, bf.module_kwargs,
                        include_bias, proj_dim=proj_dim, proj_seed=proj_seed, **proj_kwargs)


def maybe_materialize_projected(seq_len: int, k_a: int, k_g: int, kappa: float = 1.0) -> bool:
    """Capture-time rule: materialize iff ``S >= kappa*k_a*k_g/(k_a+k_g)``
    (projection.py:846-874)."""
    denom = k_a + k_g
    if denom <= 0:
        return False
    return seq_len >= kappa * (k_a * k_g) / denom


def should_materialize(capture_style: str, seq_len: int, k_a: int, k_g: int) -> bool:
    """projection.py:877-899."""
    if capture_style == "factorized":
        return False
    if capture_style == "materialized":
        return True
    if capture_style != "auto":
        raise ValueError(f"capture_style must be one of {CAPTURE_STYLES}, got {capture_style!r}.")
    return maybe_materialize_projected(seq_len, k_a, k_g)


def project_factorized(f, layer_type: str, projector, *, proj_dim: int, include_bias: bool = True,
                       proj_seed: int = 0, **proj_kwargs):
    bf = f.as_batch_first()
    return project_factors(bf.activation, bf.pre_activation_grad, layer_type, projector, bf.module_kwargs,
                           include_bias, proj_dim=proj_dim, proj_seed=proj_seed, **proj_kwargs)


def project_layer(f, layer_type: str, projector, *, style: str = "logra", capture_style: str = "factorized",
                  **proj_kwargs):
    """Route one layer through a projection style (projection.py:902-944):
    ``(payload, is_factorized)``.

    ``"logra"`` keeps ``(a_p, g_p)`` or -- when :func:`should_materialize`
    says so -- returns the ``(B, k_g*k_a)`` block from the fused kernel;
    ``"dense"`` projects the per-sample gradient; ``"mask"`` keeps fixed
    coordinates of it.  A dense input takes the ``"dense"`` path unless masked."""
    if style not in PROJECTION_STYLES:
        raise ValueError(f"style must be one of {PROJECTION_STYLES}, got {style!r}.")
    if style == "mask":
        return mask_factorized(f, layer_type, projector, **proj_kwargs), False
    if style == "dense" or isinstance(f, torch.Tensor):
        return project_materialized(f, layer_type, projector, **proj_kwargs), False
    bf = f.as_batch_first()
    a, g = bf.activation, bf.pre_activation_grad
    seq_len = a.shape[1] if a.ndim >= 3 else 1
    proj_dim = proj_kwargs["proj_dim"]
    include_bias = proj_kwargs.pop("include_bias", True)
    bias = bool(bf.module_kwargs is not None and bf.module_kwargs["has_bias"] and include_bias)
    if should_materialize(capture_style, seq_len, proj_dim, proj_dim):
        kw = dict(proj_kwargs)
        dim, seed = kw.pop("proj_dim"), kw.pop("proj_seed", 0)
        mk = {"has_bias": bias}
        return project_outer_factors(a, g, layer_type, projector, mk, True, proj_dim=dim,
                                     proj_seed=seed, **kw), False
    a_p, g_p = project_factorized(f, layer_type, projector, include_bias=include_bias, **proj_kwargs)
    return (a_p, g_p), True
