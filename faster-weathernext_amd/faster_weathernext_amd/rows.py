"""Hilbert-order gather and scatter of the node features, fused with the layer norms next to them.

The reference's patched transformer permutes the mesh nodes into Hilbert order before its
layers and back after them (``patch.py:274-276, 288-292``):

    node_features = jnp.take(node_features, perm, axis=1)      # before the layer loop
    ...                                                         # block 0 starts with st.layernorm
    x = st.layernorm(x, create_scale=False, create_offset=False)
    x = LinearNormConditioning(...)(x, norm_conditioning=...)   # per-member scale and offset
    x = jnp.take(x, argsort(perm), axis=1)                      # after the layer loop

``gather_layer_norm`` does the first gather together with block 0's layer norm, and
``layer_norm_scatter`` the final layer norm, its per-member affine and the scatter, each as one
HIP pass over [batch, n, channels] (``include/fwn_rows.h``). ``layer_norm_affine`` is the same
pass without a permutation: each block's conditioned layer norm in front of the attention and
the feed-forward (``patch.py:240-244, 250-251``), and ``add_layer_norm_affine`` adds the
residual in front of it in the same pass. The affine's scale and offset come
from the conditioning vector through LinearNormConditioning's own projections, which the caller
evaluates: pass ``mul`` (its multiplier of the normalised features) and ``add``.

The forward passes run on the GPU only. Their gradients are computed with torch operations on
the same device (the gather's transpose is the scatter and vice versa, plus the layer norm's
analytic backward).
"""
import torch

from . import _native as nat

_DTYPES = {torch.float32: nat.F32, torch.bfloat16: nat.BF16}


def _desc(x, eps):
  if not isinstance(x, torch.Tensor) or not x.is_cuda:
    raise ValueError("x must be a CUDA tensor")
  if x.dim() != 3:
    raise ValueError(f"x must be [batch, n, channels], got shape {tuple(x.shape)}")
  if x.dtype not in _DTYPES:
    raise TypeError(f"x must be float32 or bfloat16, got {x.dtype}")
  if not x.is_contiguous():
    raise ValueError("x must be contiguous")
  b, n, c = x.shape
  return nat.RowsDesc(b, n, c, _DTYPES[x.dtype], float(eps))


def _perm(perm, x):
  if not isinstance(perm, torch.Tensor) or perm.device != x.device or perm.dtype != torch.int64:
    raise ValueError("perm must be an int64 tensor on the device of x")
  if perm.shape != (x.shape[1],) or not perm.is_contiguous():
    raise ValueError(f"perm must be contiguous with shape ({x.shape[1]},), got {tuple(perm.shape)}")
  return perm


def _affine(t, x, name):
  if t is None:
    return None
  if not isinstance(t, torch.Tensor) or t.device != x.device or t.dtype != torch.float32:
    raise ValueError(f"{name} must be a float32 tensor on the device of x")
  if t.shape != (x.shape[0], x.shape[2]) or not t.is_contiguous():
    raise ValueError(f"{name} must be contiguous [batch, channels] = {(x.shape[0], x.shape[2])}")
  return t


def _stream(x):
  return torch.cuda.current_stream(x.device).cuda_stream


def _addr(t):
  return t.data_ptr() if t is not None and t.numel() else None


def gather_layer_norm_forward(x, perm, eps=1e-5, norm=True):
  """(x[:, perm], layer_norm(x[:, perm]) or None), computed by one HIP pass (no autograd)."""
  d = _desc(x, eps)
  perm = _perm(perm, x)
  x_out = torch.empty_like(x)
  n_out = torch.empty_like(x) if norm else None
  with torch.cuda.device(x.device):
    nat.check(nat.lib().fwn_rows_gather_norm_launch(d, _addr(x), _addr(perm), _addr(x_out), _addr(n_out),
                                                    _stream(x)))
  return x_out, n_out


def layer_norm_scatter_forward(x, perm, mul=None, add=None, eps=1e-5):
  """out with out[:, perm] = layer_norm(x) * mul[:, None] + add[:, None], one HIP pass (no autograd)."""
  d = _desc(x, eps)
  perm = _perm(perm, x)
  mul = _affine(mul, x, "mul")
  add = _affine(add, x, "add")
  out = torch.empty_like(x)
  with torch.cuda.device(x.device):
    nat.check(nat.lib().fwn_rows_norm_scatter_launch(d, _addr(x), _addr(perm), _addr(mul), _addr(add), _addr(out),
                                                     _stream(x)))
  return out


def layer_norm_affine_forward(x, mul=None, add=None, eps=1e-5):
  """layer_norm(x) * mul[:, None] + add[:, None], one HIP pass (no autograd)."""
  d = _desc(x, eps)
  mul = _affine(mul, x, "mul")
  add = _affine(add, x, "add")
  out = torch.empty_like(x)
  with torch.cuda.device(x.device):
    nat.check(nat.lib().fwn_rows_norm_affine_launch(d, _addr(x), _addr(mul), _addr(add), _addr(out), _stream(x)))
  return out


def add_layer_norm_affine(x, y, *, mul=None, add=None, eps=1e-5, inplace=False):
  """(x + y, layer_norm(x + y) * mul[:, None] + add[:, None]) in one HIP pass: a block's residual
  add fused with the conditioned layer norm that reads it (``patch.py:240-253``). The sum is
  added in float32 and rounded once to x's dtype, as ``x + y`` stores it, and the norm is the
  sum's. With ``inplace`` the sum is written into x. mul and add are float32 [batch, channels]
  (None: 1 and 0). Forward only: it refuses inputs that autograd would need to differentiate."""
  if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (x, y, mul, add)):
    raise RuntimeError("add_layer_norm_affine has no derivative; use x + y and layer_norm_affine under autograd")
  d = _desc(x, eps)
  if not isinstance(y, torch.Tensor) or y.shape != x.shape or y.dtype != x.dtype or y.device != x.device:
    raise ValueError("y must be a tensor of x's shape, dtype and device")
  if not y.is_contiguous():
    raise ValueError("y must be contiguous")
  mul = _affine(mul, x, "mul")
  add = _affine(add, x, "add")
  s = x if inplace else torch.empty_like(x)
  out = torch.empty_like(x)
  with torch.cuda.device(x.device):
    nat.check(nat.lib().fwn_rows_add_norm_affine_launch(d, _addr(x), _addr(y), _addr(mul), _addr(add), _addr(s),
                                                        _addr(out), _stream(x)))
  return s, out


def _norm_stats(x, eps):
  xf = x.float()
  mean = xf.mean(-1, keepdim=True)
  var = (xf - mean).square().mean(-1, keepdim=True)
  rstd = torch.rsqrt(var + eps)
  return (xf - mean) * rstd, rstd


def _norm_backward(xhat, rstd, g):
  """Gradient of layer_norm (no affine) at normalised values xhat for upstream gradient g."""
  g = g.float()
  return rstd * (g - g.mean(-1, keepdim=True) - xhat * (g * xhat).mean(-1, keepdim=True))


def _inverse(perm):
  inv = torch.empty_like(perm)
  inv[perm] = torch.arange(perm.numel(), device=perm.device)
  return inv


class _GatherNorm(torch.autograd.Function):
  @staticmethod
  def forward(ctx, x, perm, eps):
    x_out, n_out = gather_layer_norm_forward(x, perm, eps)
    ctx.save_for_backward(x_out, perm)
    ctx.eps = eps
    return x_out, n_out

  @staticmethod
  def backward(ctx, g_x, g_n):
    x_out, perm = ctx.saved_tensors
    g = torch.zeros(x_out.shape, device=x_out.device, dtype=torch.float32)
    if g_x is not None:
      g += g_x.float()
    if g_n is not None:
      xhat, rstd = _norm_stats(x_out, ctx.eps)
      g += _norm_backward(xhat, rstd, g_n)
    return g[:, _inverse(perm)].to(x_out.dtype), None, None


class _NormScatter(torch.autograd.Function):
  @staticmethod
  def forward(ctx, x, perm, mul, add, eps):
    if perm is None:
      out = layer_norm_affine_forward(x, mul, add, eps)
    else:
      out = layer_norm_scatter_forward(x, perm, mul, add, eps)
    ctx.save_for_backward(x, perm, mul)
    ctx.eps = eps
    ctx.has_add = add is not None
    return out

  @staticmethod
  def backward(ctx, g_out):
    x, perm, mul = ctx.saved_tensors
    g_y = (g_out if perm is None else g_out[:, perm]).float()  # gradient of the un-scattered rows
    xhat, rstd = _norm_stats(x, ctx.eps)
    g_mul = (g_y * xhat).sum(1) if mul is not None and ctx.needs_input_grad[2] else None
    g_add = g_y.sum(1) if ctx.has_add and ctx.needs_input_grad[3] else None
    g_xhat = g_y * mul[:, None, :] if mul is not None else g_y
    g_x = _norm_backward(xhat, rstd, g_xhat).to(x.dtype)
    return g_x, None, g_mul, g_add, None


def gather_layer_norm(x, perm, *, eps=1e-5):
  """x [batch, n, channels] -> (x[:, perm], layer_norm(x[:, perm])): the Hilbert gather before
  the layer loop (``patch.py:274-276``) and block 0's ``st.layernorm(x, create_scale=False,
  create_offset=False)`` (``patch.py:244``) in one pass. Differentiable in x."""
  return _GatherNorm.apply(x, perm, float(eps))


def layer_norm_scatter(x, perm, *, mul=None, add=None, eps=1e-5):
  """x [batch, n, channels] -> out with out[:, perm] = layer_norm(x) * mul[:, None] + add[:, None]:
  the final layer norm, LinearNormConditioning's per-member affine and the scatter back to mesh
  order (``patch.py:288-292``) in one pass. mul and add are float32 [batch, channels] (None: 1
  and 0). Differentiable in x, mul and add."""
  return _NormScatter.apply(x, perm, mul, add, float(eps))


def layer_norm_affine(x, *, mul=None, add=None, eps=1e-5):
  """x [batch, n, channels] -> layer_norm(x) * mul[:, None] + add[:, None] in one pass: a block's
  ``norm_conditioning_layer(st.layernorm(x, create_scale=False, create_offset=False))``
  (``patch.py:240-244, 250-251``). mul and add are float32 [batch, channels] (None: 1 and 0).
  Differentiable in x, mul and add."""
  return _NormScatter.apply(x, None, mul, add, float(eps))
