"""Per-sample batch normalisation of sparse features (``sparsetriton/nn/functional/norm.py:20-112``).

``sparse_batch_norm`` keeps the reference's signature and semantics: in
training each channel of each sample (rows with the same ``coords[:, 0]``) is
normalised by that sample's mean and biased variance, and the running
statistics move by ``momentum`` towards the mean over the batch's samples of
those statistics; in evaluation the running statistics are used.  Affine
``weight`` / ``bias`` are optional.

``sparse_batch_norm_act`` is the same normalisation with the residual add and
ReLU of the reference's blocks (``nn/modules/blocks.py:21-124``) fused into its
output pass: ``act(bn(x) + residual)``.

Both run as HIP kernels (``st_bn_forward`` / ``st_bn_backward``): two
deterministic statistics passes and one output pass forward, one statistics
pass and one gradient pass backward, each autograd-differentiable in the
features, the residual and the affine parameters.
"""

import ctypes
from typing import Optional

import torch

from sparsetriton_amd import _lib
from sparsetriton_amd.tensor import SparseTensor

__all__ = ["sparse_batch_norm", "sparse_batch_norm_act"]


def _f32(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if t is None:
        return None
    return t.detach().to(torch.float32).contiguous()


def _workspace(n: int, C: int, B: int, device) -> torch.Tensor:
    floats = ctypes.c_int64()
    _lib.call("st_bn_workspace", n, C, B, ctypes.byref(floats))
    return torch.empty((floats.value,), dtype=torch.float32, device=device)


class _BatchNormAct(torch.autograd.Function):
    """out = act(bn(feats) + residual); statistics per sample in training."""

    @staticmethod
    def forward(ctx, feats, weight, bias, residual, coords, batch_size, running_mean, running_var, training, eps,
                momentum, relu):
        _lib.require_device(feats, "SparseTensor features")
        x = feats.contiguous()
        n, C = x.shape
        dev = x.device
        B = max(int(batch_size), 1)
        if B > 4096:
            raise ValueError(f"sparse batch norm supports at most 4096 samples per batch (got {B})")
        res = residual.contiguous() if residual is not None else None
        if res is not None and (res.shape != x.shape or res.dtype != x.dtype):
            raise ValueError("the residual must match the features' shape and dtype")
        w32, b32 = _f32(weight), _f32(bias)
        out = torch.empty_like(x)
        s = _lib.stream_of(dev)
        if training:
            mean = torch.empty((B, C), dtype=torch.float32, device=dev)
            invstd = torch.empty((B, C), dtype=torch.float32, device=dev)
            counts = torch.empty((B,), dtype=torch.int32, device=dev)
            ws = _workspace(n, C, B, dev)
            rm = rv = None
            if running_mean is not None:
                rm = running_mean if running_mean.dtype == torch.float32 and running_mean.is_contiguous() else \
                    running_mean.float().contiguous()
            if running_var is not None:
                rv = running_var if running_var.dtype == torch.float32 and running_var.is_contiguous() else \
                    running_var.float().contiguous()
            _lib.call("st_bn_forward", _lib.ptr(x), n, C, _lib.feat_code(x.dtype), _lib.ptr(coords),
                      _lib.coord_code(coords.dtype), B, _lib.ptr(w32), _lib.ptr(b32), _lib.ptr(res), int(relu), 1,
                      float(eps), float(momentum), _lib.ptr(rm), _lib.ptr(rv), _lib.ptr(mean), _lib.ptr(invstd),
                      _lib.ptr(counts), _lib.ptr(ws), ws.numel(), _lib.ptr(out), s)
            if rm is not None and rm is not running_mean:
                running_mean.copy_(rm)
            if rv is not None and rv is not running_var:
                running_var.copy_(rv)
        else:
            if running_mean is None or running_var is None:
                raise ValueError("evaluation-mode batch norm needs running_mean and running_var")
            mean = torch.empty((C,), dtype=torch.float32, device=dev)
            invstd = torch.empty((C,), dtype=torch.float32, device=dev)
            counts = None
            rm32, rv32 = _f32(running_mean), _f32(running_var)
            _lib.call("st_bn_forward", _lib.ptr(x), n, C, _lib.feat_code(x.dtype), _lib.ptr(coords),
                      _lib.coord_code(coords.dtype), B, _lib.ptr(w32), _lib.ptr(b32), _lib.ptr(res), int(relu), 0,
                      float(eps), float(momentum), _lib.ptr(rm32), _lib.ptr(rv32), _lib.ptr(mean),
                      _lib.ptr(invstd), None, None, 0, _lib.ptr(out), s)
        # the output is needed only for the ReLU mask (so an in-place op on a plain output stays legal)
        ctx.save_for_backward(x, out if relu else None, coords, w32, mean, invstd, counts)
        ctx.meta = (B, bool(training), bool(relu), residual is not None, weight, bias)
        return out

    @staticmethod
    def backward(ctx, dout):
        x, out, coords, w32, mean, invstd, counts = ctx.saved_tensors
        B, training, relu, has_res, weight, bias = ctx.meta
        n, C = x.shape
        dev = x.device
        g = dout.contiguous()
        if g.dtype != x.dtype:
            g = g.to(x.dtype)
        need_x = ctx.needs_input_grad[0]
        dx = torch.empty_like(x)
        dres = torch.empty_like(x) if (has_res and ctx.needs_input_grad[3]) else None
        dw = torch.empty((C,), dtype=torch.float32, device=dev) if (weight is not None and ctx.needs_input_grad[1]) \
            else None
        db = torch.empty((C,), dtype=torch.float32, device=dev) if (bias is not None and ctx.needs_input_grad[2]) \
            else None
        ws = _workspace(n, C, B if training else 1, dev)
        _lib.call("st_bn_backward", _lib.ptr(x), _lib.ptr(out), _lib.ptr(g), n, C, _lib.feat_code(x.dtype),
                  _lib.ptr(coords), _lib.coord_code(coords.dtype), B, _lib.ptr(w32), int(relu), int(training),
                  _lib.ptr(mean), _lib.ptr(invstd), _lib.ptr(counts), _lib.ptr(ws), ws.numel(), _lib.ptr(dx),
                  _lib.ptr(dres), _lib.ptr(dw), _lib.ptr(db), _lib.stream_of(dev))
        dw = dw.to(weight.dtype) if dw is not None else None
        db = db.to(bias.dtype) if db is not None else None
        return (dx if need_x else None, dw, db, dres, None, None, None, None, None, None, None, None)


def sparse_batch_norm_act(
    tensor: SparseTensor,
    weight: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    running_mean: Optional[torch.Tensor] = None,
    running_var: Optional[torch.Tensor] = None,
    training: bool = True,
    eps: float = 1e-5,
    momentum: float = 0.1,
    residual: Optional[torch.Tensor] = None,
    relu: bool = False,
) -> SparseTensor:
    """``act(bn(tensor.F) + residual)`` as one kernel pass (``act`` = ReLU or identity)."""
    if tensor.F.dim() != 2:
        raise ValueError(f"Expected 2D input, got {tensor.F.dim()}D")
    feats = _BatchNormAct.apply(tensor.F, weight, bias, residual, tensor.C.contiguous(), tensor.batch_size,
                                running_mean, running_var, bool(training), float(eps), float(momentum), bool(relu))
    return tensor.replace(feats)


def sparse_batch_norm(
    tensor: SparseTensor,
    weight: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    running_mean: Optional[torch.Tensor] = None,
    running_var: Optional[torch.Tensor] = None,
    training: bool = True,
    eps: float = 1e-5,
    momentum: float = 0.1,
) -> SparseTensor:
    """Per-sample batch normalisation (reference ``norm.py:20-112``)."""
    return sparse_batch_norm_act(tensor, weight, bias, running_mean, running_var, training, eps, momentum)
