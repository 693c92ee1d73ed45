"""Math-engine drop-in: the residual-VQ weight container, its code packing and
the multi-stage subspace LUT GEMM, on the HIP kernels of csrc/lut_rvq.hip.

Mirrors ojasx_24x96/codec.py:77-214 (QuantizedWeight, pack_codes,
unpack_codes) and ojasx_24x96/math_engine.py:136-208 (subspace_lut_rvq_gemm):
same names, argument meaning, validation and errors.  Computation runs on the
GPU only; CPU tensors raise.  The container itself is plain validation and
accepts tensors on any device.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, Optional, Tuple

from . import _lib

_SUPPORTED_WIDTHS = (1, 2, 4, 8)


def _torch():
    import torch
    return torch


def _vp(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    torch = _torch()
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _require_gpu(t, what):
    if not t.is_cuda:
        raise RuntimeError(f"{what}: the LUT engine runs on the GPU only (got a {t.device} tensor)")


@dataclass
class QuantizedWeight:
    """Portable encoded representation of one rank-two weight matrix
    (codec.py:77-174): ``stages`` residual stages, each a packed stream of
    ``rows * ceil(columns / block_size)`` codes of ``bits_per_stage`` bits and a
    ``[2^bits, block_size]`` fp32 codebook, plus fp32 row scales."""

    original_shape: Tuple[int, int]
    block_size: int
    bits_per_stage: int
    packed_codes: "torch.Tensor"
    codebooks: "torch.Tensor"
    row_scales: "torch.Tensor"
    metrics: Dict[str, object] = field(default_factory=dict)

    def __post_init__(self) -> None:
        torch = _torch()
        if len(self.original_shape) != 2:
            raise ValueError("Only rank-two weights are supported")
        if self.bits_per_stage not in _SUPPORTED_WIDTHS:
            raise ValueError("Unsupported code width")
        if self.packed_codes.dtype != torch.uint8:
            raise TypeError("packed_codes must be uint8")
        if self.codebooks.dtype != torch.float32 or self.row_scales.dtype != torch.float32:
            raise TypeError("Codebooks and scales use float32 storage")
        if self.packed_codes.device != self.codebooks.device or (
                self.packed_codes.device != self.row_scales.device):
            raise ValueError("All encoded tensors must be on one device")
        rows, columns = self.original_shape
        if rows < 0 or columns < 0:
            raise ValueError("Weight dimensions must be nonnegative")
        blocks_per_row = (columns + self.block_size - 1) // self.block_size
        vectors = rows * blocks_per_row
        if self.codebooks.ndim != 3:
            raise ValueError("Codebooks must be a rank-three tensor")
        stages = self.codebooks.shape[0]
        if stages < 1:
            raise ValueError("An encoded weight requires at least one residual stage")
        expected_packed = (vectors * self.bits_per_stage + 7) // 8
        if tuple(self.codebooks.shape[1:]) != (1 << self.bits_per_stage, self.block_size):
            raise ValueError("Codebook shape is inconsistent with the codec")
        if tuple(self.packed_codes.shape) != (stages, expected_packed):
            raise ValueError("Packed-code shape is inconsistent with the weight shape")
        if tuple(self.row_scales.shape) != (rows,):
            raise ValueError("Row-scale shape is inconsistent with the weight shape")

    @property
    def stages(self) -> int:
        return int(self.codebooks.shape[0])

    @property
    def blocks_per_row(self) -> int:
        return (self.original_shape[1] + self.block_size - 1) // self.block_size

    @property
    def vector_count(self) -> int:
        return self.original_shape[0] * self.blocks_per_row

    @property
    def storage_bytes(self) -> int:
        return (self.packed_codes.numel()
                + self.codebooks.numel() * self.codebooks.element_size()
                + self.row_scales.numel() * self.row_scales.element_size())

    @property
    def nominal_bits_per_weight(self) -> float:
        return self.stages * self.bits_per_stage / self.block_size

    @property
    def measured_bits_per_weight(self) -> float:
        elements = self.original_shape[0] * self.original_shape[1]
        return 8.0 * self.storage_bytes / elements if elements else 0.0

    def codes(self, stage: int):
        if not 0 <= stage < self.stages:
            raise IndexError("Invalid residual stage")
        return unpack_codes(self.packed_codes[stage], self.bits_per_stage, self.vector_count)

    def codes_range(self, stage: int, start: int, count: int):
        """Unpack a bounded logical code range, including unaligned bit offsets."""
        torch = _torch()
        if not 0 <= stage < self.stages:
            raise IndexError("Invalid residual stage")
        if start < 0 or count < 0 or start + count > self.vector_count:
            raise IndexError("Invalid logical code range")
        if count == 0:
            return torch.empty(0, dtype=torch.uint8, device=self.packed_codes.device)
        bits = self.bits_per_stage
        per_byte = 8 // bits
        first_byte = (start * bits) // 8
        final_byte = ((start + count) * bits + 7) // 8
        window = self.packed_codes[stage, first_byte:final_byte]
        window_codes = unpack_codes(window, bits, window.numel() * per_byte)
        offset = start - first_byte * per_byte
        return window_codes[offset:offset + count]


def pack_codes(codes, bits: int):
    """Pack unsigned codes using a deterministic little-endian bit order
    (codec.py:176-195), on the GPU."""
    torch = _torch()
    if bits not in _SUPPORTED_WIDTHS:
        raise ValueError("Only 1-, 2-, 4-, and 8-bit codes are supported")
    if codes.dtype not in (torch.uint8, torch.int16, torch.int32, torch.int64):
        raise TypeError("Codes must have an integer dtype")
    _require_gpu(codes, "pack_codes")
    flat = codes.reshape(-1)
    if flat.numel() and (flat.min().item() < 0 or flat.max().item() >= (1 << bits)):
        raise ValueError("A code exceeds the requested bit width")
    flat8 = flat.to(dtype=torch.uint8).contiguous()
    out = torch.empty((flat8.numel() * bits + 7) // 8, dtype=torch.uint8, device=codes.device)
    _lib.check(_lib.lib().ojasx_pack_codes_device(_vp(flat8), flat8.numel(), bits, _vp(out),
                                                   _stream()), "ojasx_pack_codes_device")
    return out


def unpack_codes(packed, bits: int, count: int):
    """Inverse of :func:`pack_codes`, with explicit logical code count
    (codec.py:198-214), on the GPU."""
    torch = _torch()
    if bits not in _SUPPORTED_WIDTHS:
        raise ValueError("Only 1-, 2-, 4-, and 8-bit codes are supported")
    if packed.dtype != torch.uint8 or count < 0:
        raise ValueError("Packed codes must be uint8 and count nonnegative")
    expected = (count * bits + 7) // 8
    if packed.numel() != expected:
        raise ValueError(f"Expected {expected} packed bytes, received {packed.numel()}")
    _require_gpu(packed, "unpack_codes")
    out = torch.empty(count, dtype=torch.uint8, device=packed.device)
    if count == 0:
        return out
    src = packed.reshape(-1).contiguous()
    _lib.check(_lib.lib().ojasx_unpack_codes_device(_vp(src), count, bits, _vp(out), _stream()),
               "ojasx_unpack_codes_device")
    return out


def subspace_lut_rvq_gemm(inputs, encoded: QuantizedWeight, bias=None, *, row_block_size: int = 256):
    """Y[b, m] = row_scales[m] * sum_{s, g} LUT[b, s, g, code_s[m, g]] + bias[m]
    with LUT[b, s, g, q] = <X[b, g, :], C[s, q, :]> and X zero-padded to whole
    blocks (math_engine.py:136-208).  Returns the input dtype and shape
    [..., rows].  ``row_block_size`` bounds the reference's gather memory and
    is accepted for interface parity; the kernel streams rows without it."""
    torch = _torch()
    rows, columns = encoded.original_shape
    if inputs.shape[-1] != columns:
        raise ValueError(f"Input feature mismatch: expected {columns}, got {inputs.shape[-1]}")
    _require_gpu(inputs, "subspace_lut_rvq_gemm")
    del row_block_size
    device = inputs.device
    orig_shape, orig_dtype = inputs.shape, inputs.dtype
    flat = inputs.reshape(-1, columns)
    if flat.dtype == torch.bfloat16:
        compute, tag = torch.bfloat16, 1
    else:
        compute, tag = torch.float32, 0
        flat = flat.to(torch.float32)
    flat = flat.contiguous()
    batch = flat.shape[0]
    y = torch.empty(batch, rows, dtype=compute, device=device)
    if batch and rows:
        packed = encoded.packed_codes.to(device=device).contiguous()
        cbs = encoded.codebooks.to(device=device, dtype=torch.float32).contiguous()
        scales = encoded.row_scales.to(device=device, dtype=torch.float32).contiguous()
        b = None
        if bias is not None:
            b = bias.to(device=device, dtype=torch.float32).contiguous()
        rc = _lib.lib().ojasx_subspace_lut_gemm_device(
            _vp(flat), batch, columns, rows, _vp(packed), packed.stride(0) if packed.dim() == 2 else 0,
            encoded.stages, encoded.bits_per_stage, encoded.block_size, _vp(cbs), _vp(scales),
            _vp(b) if b is not None else None, _vp(y), tag, _stream())
        _lib.check(rc, "ojasx_subspace_lut_gemm_device")
    return y.to(dtype=orig_dtype).reshape(*orig_shape[:-1], rows)
