"""PyTorch module face: ``SplitManifoldLUTLinear`` with the reference's API
(split_manifold_lut_experiment/engine/split_manifold_engine.py:22-267),
executed by the HIP C-ABI library on the tensor's GPU.

Same constructor arguments, buffers (``codebook`` [Kcb, D], ``codes`` [M, G]
uint8, ``scales`` [M], ``outlier_indices`` [2, nnz] int64 COO row-major,
``outlier_values`` [nnz]), optional ``bias`` parameter, properties
(``lut_sram_bytes``, ``compression_ratio``) and methods (``from_dense``,
``build_lut``, ``forward``, ``dequantize_weights``).

Execution: ``forward`` and ``build_lut`` require CUDA (ROCm) tensors and the
built library; there is no CPU fallback.  On first use (and whenever a buffer
changes) the buffers are copied once into a device-resident native handle that
holds the codes repacked into the kernel's tile layout and the outliers as
per-slice buckets; ``forward`` then launches one fused kernel on the current
stream.  fp32 and bf16 activations are supported; the LUT and all sums are
fp32 internally (the reference computes bf16 layers in bf16, so bf16 results
agree to the bf16 tolerance).
"""
import ctypes
import math
from typing import Optional

import torch
import torch.nn as nn

from ._lib import DTYPE_BF16, DTYPE_F32, check, lib


def _dtype_tag(dt):
    if dt == torch.float32:
        return DTYPE_F32
    if dt == torch.bfloat16:
        return DTYPE_BF16
    raise TypeError(f"unsupported activation dtype {dt}; use float32 or bfloat16")


def _stream_ptr(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_gpu(t, what):
    if not t.is_cuda:
        raise RuntimeError(f"{what}: the LUT engine runs on the GPU only; got a {t.device} "
                           "tensor (move the module and inputs to a ROCm device)")


class SplitManifoldLUTLinear(nn.Module):
    """split_manifold_engine.py:22-69 (constructor, buffers, asserts)."""

    def __init__(self, in_features: int, out_features: int, block_dim: int = 16,
                 codebook_size: int = 256, outlier_tau: float = 3.5, bias: bool = False,
                 dtype: torch.dtype = torch.float32):
        super().__init__()
        assert in_features % block_dim == 0, (
            f"in_features ({in_features}) must be divisible by block_dim ({block_dim})")
        assert codebook_size <= 256, "codebook_size must fit in uint8 (<= 256)"
        self.in_features = in_features
        self.out_features = out_features
        self.block_dim = block_dim
        self.num_groups = in_features // block_dim
        self.codebook_size = codebook_size
        self.outlier_tau = outlier_tau
        self.dtype = dtype
        self.register_buffer("codebook", torch.zeros((codebook_size, block_dim), dtype=dtype))
        self.register_buffer("codes", torch.zeros((out_features, self.num_groups), dtype=torch.uint8))
        self.register_buffer("scales", torch.ones(out_features, dtype=dtype))
        self.register_buffer("outlier_indices", torch.empty((2, 0), dtype=torch.long))
        self.register_buffer("outlier_values", torch.empty((0,), dtype=dtype))
        self.num_outliers = 0
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=dtype))
        else:
            self.register_parameter("bias", None)
        self._native = None
        self._native_key = None

    # -- properties: split_manifold_engine.py:71-88 --------------------------
    @property
    def lut_sram_bytes(self) -> int:
        elem = 4 if self.dtype in (torch.float32, torch.int32) else 2
        return self.num_groups * self.codebook_size * elem

    @property
    def compression_ratio(self) -> float:
        dense = self.out_features * self.in_features * 2
        comp = (self.out_features * self.num_groups + self.codebook_size * self.block_dim * 2
                + self.out_features * 2 + self.num_outliers * (8 + 2))
        return dense / max(1, comp)

    # -- offline encoder: split_manifold_engine.py:90-183 ---------------------
    @classmethod
    def from_dense(cls, dense_weight: torch.Tensor, dense_bias: Optional[torch.Tensor] = None,
                   block_dim: int = 16, codebook_size: int = 256,
                   outlier_tau: float = 3.5) -> "SplitManifoldLUTLinear":
        """Offline fit (not on the hot path): outliers |W - mean| >= tau*std,
        per-row max-abs scales, 5 Lloyd iterations from evenly spaced samples,
        nearest-centroid codes, exact residual outliers.  Runs with torch on the
        weight's device."""
        out_f, in_f = dense_weight.shape
        layer = cls(in_f, out_f, block_dim, codebook_size, outlier_tau,
                    bias=dense_bias is not None, dtype=dense_weight.dtype)
        with torch.no_grad():
            W = dense_weight.detach().clone().float()
            thr = outlier_tau * W.std().item()
            mask = (W - W.mean().item()).abs() >= thr
            idx = torch.nonzero(mask, as_tuple=False).t()
            Wm = W.clone()
            Wm[mask] = 0.0
            G = in_f // block_dim
            blocks = Wm.view(out_f, G, block_dim)
            rs = blocks.abs().amax(dim=(1, 2), keepdim=True).clamp(min=1e-8)
            vecs = (blocks / rs).reshape(-1, block_dim)
            pick = torch.linspace(0, vecs.shape[0] - 1, codebook_size, dtype=torch.long,
                                  device=vecs.device)
            cents = vecs[pick].clone()
            for _ in range(5):
                ids = torch.cdist(vecs, cents).argmin(dim=1)
                acc = torch.zeros_like(cents).index_add_(0, ids, vecs)
                cnt = torch.zeros(codebook_size, device=cents.device).index_add_(
                    0, ids, torch.ones_like(ids, dtype=torch.float32))
                ok = cnt > 0
                cents[ok] = acc[ok] / cnt[ok].unsqueeze(1)
            best = torch.cdist(vecs, cents).argmin(dim=1).view(out_f, G)
            What = (cents[best] * rs).reshape(out_f, in_f)
            layer.scales = rs.view(out_f).to(dense_weight.dtype)
            layer.codebook = cents.to(dense_weight.dtype)
            layer.codes = best.to(torch.uint8)
            layer.outlier_indices = idx
            layer.outlier_values = (W - What)[mask].to(dense_weight.dtype)
            layer.num_outliers = layer.outlier_values.numel()
            if dense_bias is not None:
                layer.bias.data.copy_(dense_bias.data)
        return layer

    # -- native handle --------------------------------------------------------
    def _key(self):
        ts = [self.codebook, self.codes, self.scales, self.outlier_indices, self.outlier_values]
        if self.bias is not None:
            ts.append(self.bias)
        return tuple((t.data_ptr(), t._version, t.device) for t in ts) + (self.num_outliers,)

    def _handle(self):
        key = self._key()
        if self._native is not None and self._native_key == key:
            return self._native
        self._release()
        import numpy as np
        L = lib()
        cb = self.codebook.detach().float().cpu().contiguous().numpy()
        cd = self.codes.detach().cpu().contiguous().numpy()
        sc = self.scales.detach().float().cpu().contiguous().numpy()
        bs = None if self.bias is None else self.bias.detach().float().cpu().contiguous().numpy()
        p = lambda a: None if a is None else a.ctypes.data_as(ctypes.c_void_p)
        dev = torch.cuda.current_device()
        torch.cuda.set_device(self.codes.device)
        try:
            h = L.ojasx_create_linear(self.in_features, self.out_features, self.block_dim,
                                      self.codebook_size, p(cb), p(cd), p(sc), p(bs))
            if not h:
                raise RuntimeError("ojasx_create_linear failed: "
                                   + L.ojasx_get_last_error().decode(errors="replace"))
            nnz = int(self.outlier_values.numel()) if self.num_outliers > 0 else 0
            if nnz:
                rows = self.outlier_indices[0].detach().cpu()
                cols = self.outlier_indices[1].detach().cpu()
                vals = self.outlier_values.detach().float().cpu()
                order = torch.argsort(rows * self.in_features + cols, stable=True)
                rows, cols, vals = rows[order], cols[order], vals[order]
                rp = torch.zeros(self.out_features + 1, dtype=torch.int64)
                rp[1:] = torch.cumsum(torch.bincount(rows, minlength=self.out_features), 0)
                rp = rp.to(torch.int32).numpy()
                cl = cols.to(torch.int32).numpy()
                vl = vals.numpy().astype(np.float32)
                rc = L.ojasx_set_linear_outliers(h, nnz, p(rp), p(cl), p(vl))
                if rc:
                    L.ojasx_destroy_linear(h)
                    check(rc, "ojasx_set_linear_outliers")
        finally:
            torch.cuda.set_device(dev)
        self._native, self._native_key = h, key
        return h

    def _release(self):
        if getattr(self, "_native", None):
            lib().ojasx_destroy_linear(self._native)
        self._native = None
        self._native_key = None

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass

    # -- hot path -------------------------------------------------------------
    def build_lut(self, x: torch.Tensor) -> torch.Tensor:
        """LUT[..., g, k] = <x_g, C[k]> (split_manifold_engine.py:185-200), by the
        HIP LUT-build kernel; fp32 result."""
        _require_gpu(x, "build_lut")
        *bd, k = x.shape
        xf = x.reshape(-1, k).contiguous()
        cb = self.codebook.to(device=x.device, dtype=torch.float32).contiguous()
        out = torch.empty(xf.shape[0], self.num_groups, self.codebook_size, device=x.device,
                          dtype=torch.float32)
        with torch.cuda.device(x.device):
            check(lib().ojasx_build_lut_device(
                ctypes.c_void_p(xf.data_ptr()), ctypes.c_void_p(cb.data_ptr()), xf.shape[0],
                self.num_groups, self.block_dim, self.codebook_size,
                ctypes.c_void_p(out.data_ptr()), _dtype_tag(xf.dtype), _stream_ptr(x.device)),
                "ojasx_build_lut_device")
        return out.view(*bd, self.num_groups, self.codebook_size)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """split_manifold_engine.py:202-250: y = s * sum_g LUT[g, codes] + outliers
        + bias, one fused kernel."""
        _require_gpu(x, "forward")
        *bd, k = x.shape
        if k != self.in_features:
            raise ValueError(f"expected last dim {self.in_features}, got {k}")
        xf = x.reshape(-1, k).contiguous()
        y = torch.empty(xf.shape[0], self.out_features, device=x.device, dtype=x.dtype)
        with torch.cuda.device(x.device):
            h = self._handle()
            check(lib().ojasx_linear_forward_device(
                h, ctypes.c_void_p(xf.data_ptr()), ctypes.c_void_p(y.data_ptr()), xf.shape[0],
                _dtype_tag(x.dtype), _stream_ptr(x.device)), "ojasx_linear_forward_device")
        return y.view(*bd, self.out_features)

    def dequantize_weights(self) -> torch.Tensor:
        """Diagnostic dense weight (split_manifold_engine.py:252-267)."""
        with torch.no_grad():
            W = (self.codebook[self.codes.long()] * self.scales.view(-1, 1, 1)).reshape(
                self.out_features, self.in_features)
            Wo = torch.zeros_like(W)
            if self.num_outliers > 0:
                Wo[self.outlier_indices[0], self.outlier_indices[1]] = self.outlier_values
            return W + Wo
