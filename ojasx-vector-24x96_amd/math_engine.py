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


def _packed_geometry(shape, block: int, bits: int):
    """(codes per row, total codes, packed bytes per stage) of a rows x columns
    weight cut into block-wide vectors, one ``bits``-wide code each."""
    rows, cols = shape
    per_row = -(-cols // block)
    count = rows * per_row
    return per_row, count, -(-count * bits // 8)


@dataclass
class QuantizedWeight:
    """Encoded rank-two weight of the residual-VQ codec (ojasx_24x96/codec.py:77-174):
    ``codebooks[s]`` is stage s's ``[2^bits, block_size]`` fp32 codebook,
    ``packed_codes[s]`` its codes (one per ``block_size``-wide vector of a row,
    rows in order, ``bits_per_stage`` bits each, little-endian within bytes),
    ``row_scales`` the fp32 scale of every row.  Field names, properties and
    exception types (ValueError for shapes, widths and devices, TypeError for
    storage dtypes, IndexError for stage and code ranges) are the reference's."""

    original_shape: Tuple[int, int]
    block_size: int
    bits_per_stage: int
    packed_codes: "torch.Tensor"
    codebooks: "torch.Tensor"
    row_scales: "torch.Tensor"
    metrics: Dict[str, object] = field(default_factory=dict)

    def __post_init__(self) -> None:
        torch = _torch()
        shape = tuple(self.original_shape)
        if len(shape) != 2 or min(shape) < 0:
            raise ValueError(f"QuantizedWeight encodes a rank-two weight with nonnegative "
                             f"dimensions, not shape {shape}")
        if self.bits_per_stage not in _SUPPORTED_WIDTHS:
            raise ValueError(f"code width {self.bits_per_stage} is not one of "
                             f"{_SUPPORTED_WIDTHS}")
        # storage dtypes first (TypeError), then one device, then the shapes
        for name, want in (("packed_codes", torch.uint8), ("codebooks", torch.float32),
                           ("row_scales", torch.float32)):
            got = getattr(self, name).dtype
            if got != want:
                raise TypeError(f"{name} is stored as {got}; the codec stores {want}")
        devices = {t.device for t in (self.packed_codes, self.codebooks, self.row_scales)}
        if len(devices) != 1:
            raise ValueError(f"encoded tensors span several devices: {sorted(map(str, devices))}")
        if self.codebooks.ndim != 3 or self.codebooks.shape[0] < 1:
            raise ValueError(f"codebooks must be [stages >= 1, 2^bits, block_size], got "
                             f"{tuple(self.codebooks.shape)}")
        _, _, nbytes = _packed_geometry(shape, self.block_size, self.bits_per_stage)
        expected = {"codebooks": (self.stages, 1 << self.bits_per_stage, self.block_size),
                    "packed_codes": (self.stages, nbytes),
                    "row_scales": (shape[0],)}
        for name, want in expected.items():
            got = tuple(getattr(self, name).shape)
            if got != want:
                raise ValueError(f"{name} has shape {got}; a {shape[0]} x {shape[1]} weight with "
                                 f"block {self.block_size} and {self.bits_per_stage}-bit codes "
                                 f"needs {want}")

    @property
    def stages(self) -> int:
        return int(self.codebooks.shape[0])

    @property
    def blocks_per_row(self) -> int:
        return _packed_geometry(self.original_shape, self.block_size, self.bits_per_stage)[0]

    @property
    def vector_count(self) -> int:
        return _packed_geometry(self.original_shape, self.block_size, self.bits_per_stage)[1]

    @property
    def storage_bytes(self) -> int:
        return sum(t.numel() * t.element_size()
                   for t in (self.packed_codes, self.codebooks, self.row_scales))

    @property
    def nominal_bits_per_weight(self) -> float:
        return self.stages * self.bits_per_stage / self.block_size

    @property
    def measured_bits_per_weight(self) -> float:
        rows, cols = self.original_shape
        return 8.0 * self.storage_bytes / (rows * cols) if rows * cols else 0.0

    def _stage(self, stage: int) -> int:
        if stage < 0 or stage >= self.stages:
            raise IndexError(f"stage {stage} outside [0, {self.stages})")
        return stage

    def codes(self, stage: int):
        """All codes of one stage, uint8, in vector order."""
        return unpack_codes(self.packed_codes[self._stage(stage)], self.bits_per_stage,
                            self.vector_count)

    def codes_range(self, stage: int, start: int, count: int):
        """Codes start .. start + count - 1 of one stage.  A byte holds
        8 / bits whole codes, so only the bytes covering the range are
        unpacked and the codes before ``start`` in its first byte dropped."""
        torch = _torch()
        s = self._stage(stage)
        if start < 0 or count < 0 or start + count > self.vector_count:
            raise IndexError(f"code range [{start}, {start + count}) outside "
                             f"[0, {self.vector_count})")
        if count == 0:
            return torch.empty(0, dtype=torch.uint8, device=self.packed_codes.device)
        per = 8 // self.bits_per_stage
        lo, hi = start // per, -(-(start + count) // per)
        unpacked = unpack_codes(self.packed_codes[s, lo:hi], self.bits_per_stage, (hi - lo) * per)
        skip = start - lo * per
        return unpacked[skip:skip + count]


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
