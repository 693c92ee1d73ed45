"""Paged KV storage on the GPU, on the kernels of csrc/kv_pages.hip and
csrc/lut_kv.hip.

* ``PagedCompressedKVCache`` mirrors ojasx_24x96/long_context.py:212-279: the
  int8 cache with per-token fp16 scales and sink + sliding-window eviction.
  Names, argument meaning, validation, the page list ``_pages`` of
  ``(qk, sk, qv, sv)`` and ``storage_bytes`` match the reference.  Pages live
  in a pool of at most ``max_resident_pages`` page buffers that is allocated as
  pages are first needed and recycled on eviction, so a long stream allocates
  nothing in steady state.  Each entry of ``_pages`` is a view of its buffer
  trimmed to the page's length; an evicted page's buffer is rewritten by a
  later page.
* ``PagedCodeKVCache`` is the code-domain counterpart for decode: per token
  and kv head, 8-bit codes into a 256-centroid codebook (or the reference's
  scalar quantiser, ojasx_lut_kv_cache.cpp:16-65) and an fp32 scale, in the
  page layout [page][kv head][slot][group] that ``decode`` reads through a
  block table.  Tokens fill pages in order; opening a page beyond
  ``max_resident_pages`` evicts the oldest page after the ``sink_pages`` first
  ones (the reference's eviction rule, long_context.py:255-257).

Everything runs on the GPU; CPU tensors raise.
"""
from __future__ import annotations

import ctypes
from typing import Iterator, List, Optional, Tuple

import numpy as np

from . import _lib


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
        raise RuntimeError(f"{what}: the KV cache runs on the GPU only (got a {t.device} tensor)")


def _dtype_tag(dtype):
    torch = _torch()
    tags = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
    if dtype not in tags:
        raise TypeError(f"unsupported KV dtype {dtype}: float32, bfloat16 or float16")
    return tags[dtype]


def _quantize_into(t, q, s):
    """Quantise t [..., R, D] (contiguous over its last two dimensions, uniform
    stride over the leading ones) into q [..., >=R, D] int8 and s [..., >=R, 1]
    fp16 views with the same leading shape."""
    lead = int(np.prod(t.shape[:-2])) if t.dim() > 2 else 1
    rows, dim = t.shape[-2], t.shape[-1]
    if rows > 2**31 - 1 or dim > 2**31 - 1:
        raise ValueError("int8 quantisation: more than 2^31 - 1 rows or columns in one call")
    xs = t.stride(-3) if t.dim() > 2 else rows * dim
    qs = q.stride(-3) if q.dim() > 2 else 0
    ss = s.stride(-3) if s.dim() > 2 else 0
    rc = _lib.lib().ojasx_quantize_int8_device(_vp(t), lead, rows, dim, xs, _dtype_tag(t.dtype),
                                               _vp(q), qs, _vp(s), ss, _stream())
    _lib.check(rc, "ojasx_quantize_int8_device")


class PagedCompressedKVCache:
    """Bounded-memory int8 paged KV cache (long_context.py:212-279): K/V pages
    of ``page_size`` tokens quantised per token to int8 with an fp16 scale;
    beyond ``max_resident_pages`` pages the oldest page after the
    ``sink_pages`` first ones is evicted."""

    def __init__(self, page_size: int = 256, max_resident_pages: int = 64,
                 sink_pages: int = 2) -> None:
        if page_size <= 0 or max_resident_pages <= sink_pages:
            raise ValueError("Invalid page configuration for PagedCompressedKVCache")
        self.page_size = int(page_size)
        self.max_resident_pages = int(max_resident_pages)
        self.sink_pages = int(sink_pages)
        self.total_tokens_seen: int = 0
        self._pages: List[Tuple] = []
        self._slots: List[int] = []      # page buffer of each resident page
        self._buffers: List[Tuple] = []  # (qk, sk, qv, sv) page buffers
        self._free: List[int] = []
        self._layout = None              # (B, H, D, device) of the first append

    @staticmethod
    def _quantize_int8(t):
        """long_context.py:234-240 on the GPU: t [..., D] float32/bfloat16/
        float16 -> (q int8 [..., D], scale float16 [..., 1])."""
        torch = _torch()
        _require_gpu(t, "PagedCompressedKVCache._quantize_int8")
        t = t.contiguous()
        q = torch.empty(t.shape, dtype=torch.int8, device=t.device)
        s = torch.empty((*t.shape[:-1], 1), dtype=torch.float16, device=t.device)
        if t.numel():
            flat = t.reshape(1, -1, t.shape[-1])
            _quantize_into(flat, q.view(1, -1, t.shape[-1]), s.view(1, -1, 1))
        return q, s

    @staticmethod
    def _dequantize_int8(q, scale, dtype):
        """long_context.py:242-244 on the GPU: float(q) * float(scale) in
        float32, returned as ``dtype``."""
        torch = _torch()
        _require_gpu(q, "PagedCompressedKVCache._dequantize_int8")
        out = torch.empty(q.shape, dtype=dtype, device=q.device)
        if q.numel():
            dim = q.shape[-1]
            qs, ss = _group_stride(q), _group_stride(scale)
            if q.dim() < 3 or qs is None or ss is None or q.stride(-1) != 1 or \
                    q.stride(-2) != dim or scale.stride(-2) != 1:
                q, scale = q.contiguous().view(1, -1, dim), scale.contiguous().view(1, -1, 1)
                qs = ss = 0
            groups, rows = q.numel() // (q.shape[-2] * dim), q.shape[-2]
            rc = _lib.lib().ojasx_dequantize_int8_device(
                _vp(q), _vp(scale), groups, rows, dim, qs, ss, _vp(out), _dtype_tag(dtype),
                _stream())
            _lib.check(rc, "ojasx_dequantize_int8_device")
        return out

    def _take_buffer(self, B, H, D, device) -> int:
        torch = _torch()
        if self._free:
            return self._free.pop()
        P = self.page_size
        qk = torch.empty(B, H, P, D, dtype=torch.int8, device=device)
        sk = torch.empty(B, H, P, 1, dtype=torch.float16, device=device)
        qv = torch.empty_like(qk)
        sv = torch.empty_like(sk)
        self._buffers.append((qk, sk, qv, sv))
        return len(self._buffers) - 1

    def append(self, key, value) -> None:
        """Quantise and append a K/V chunk ``[B, H, S, D]`` into bounded pages
        (long_context.py:246-257)."""
        _require_gpu(key, "PagedCompressedKVCache.append")
        _require_gpu(value, "PagedCompressedKVCache.append")
        if key.dim() != 4 or key.shape != value.shape:
            raise ValueError("key and value must both be [B, H, S, D] of one shape")
        B, H, S, D = key.shape
        layout = (B, H, D, key.device)
        if self._layout is None:
            self._layout = layout
        elif layout != self._layout:
            raise ValueError(f"chunk layout {layout[:3]} differs from the cache's {self._layout[:3]}")
        self.total_tokens_seen += S
        key, value = key.contiguous(), value.contiguous()
        for start in range(0, S, self.page_size):
            n = min(start + self.page_size, S) - start
            if len(self._pages) == self.max_resident_pages:
                # Evicting before the append leaves the same pages as the
                # reference's append-then-pop(sink_pages), with one page
                # buffer fewer.
                self._pages.pop(self.sink_pages)
                self._free.append(self._slots.pop(self.sink_pages))
            slot = self._take_buffer(B, H, D, key.device)
            qk, sk, qv, sv = self._buffers[slot]
            _quantize_into(key[:, :, start:start + n], qk, sk)
            _quantize_into(value[:, :, start:start + n], qv, sv)
            self._pages.append((qk[:, :, :n], sk[:, :, :n], qv[:, :, :n], sv[:, :, :n]))
            self._slots.append(slot)

    def iter_dequantized_pages(self, dtype=None) -> Iterator[Tuple]:
        """Lazily dequantise resident pages one by one (long_context.py:259-267)."""
        torch = _torch()
        dtype = torch.float32 if dtype is None else dtype
        for qk, sk, qv, sv in self._pages:
            yield (self._dequantize_int8(qk, sk, dtype), self._dequantize_int8(qv, sv, dtype))

    @property
    def resident_tokens(self) -> int:
        return sum(p[0].shape[2] for p in self._pages)

    @property
    def storage_bytes(self) -> int:
        total = 0
        for page in self._pages:
            for t in page:
                total += t.numel() * t.element_size()
        return total


def _group_stride(t):
    """Element stride between consecutive [rows, last] matrices of t when its
    leading dimensions collapse into one, else None."""
    if t.dim() < 3:
        return 0
    gs = t.stride(-3)
    expect = gs * t.shape[-3]
    for i in range(t.dim() - 4, -1, -1):
        if t.shape[i] > 1 and t.stride(i) != expect:
            return None
        expect *= t.shape[i]
    return gs


class PageTable:
    """Host bookkeeping of a token-filled paged cache with sink + sliding
    eviction: logical pages in order (``pages``, physical ids), tokens in the
    last page (``tail``) and the free physical pages.  ``plan(n)`` places n
    new tokens and returns each token's slot (page * page_size + offset), -1
    for a token whose page is evicted again within the same call."""

    def __init__(self, page_size: int, max_pages: int, sink_pages: int) -> None:
        if page_size <= 0 or max_pages <= sink_pages or sink_pages < 0:
            raise ValueError("Invalid page configuration for PagedCodeKVCache")
        self.page_size = page_size
        self.max_pages = max_pages
        self.sink_pages = sink_pages
        self.pages: List[int] = []
        self._gen: List[int] = []
        self._next_gen = 0
        self.tail = 0
        self._free = list(range(max_pages - 1, -1, -1))

    @property
    def seq_len(self) -> int:
        return (len(self.pages) - 1) * self.page_size + self.tail if self.pages else 0

    def _open_page(self) -> None:
        if len(self.pages) == self.max_pages:
            self._free.append(self.pages.pop(self.sink_pages))
            self._gen.pop(self.sink_pages)
        self.pages.append(self._free.pop())
        self._gen.append(self._next_gen)
        self._next_gen += 1
        self.tail = 0

    def plan(self, n: int) -> np.ndarray:
        P = self.page_size
        slots = np.empty(n, np.int32)
        gens = np.empty(n, np.int64)
        t = 0
        while t < n:
            if not self.pages or self.tail == P:
                self._open_page()
            m = min(P - self.tail, n - t)
            slots[t:t + m] = self.pages[-1] * P + self.tail + np.arange(m, dtype=np.int32)
            gens[t:t + m] = self._gen[-1]
            self.tail += m
            t += m
        slots[~np.isin(gens, np.asarray(self._gen, np.int64))] = -1
        return slots


class PagedCodeKVCache:
    """Code-domain paged KV cache of one attention layer on the GPU.

    ``append(k, v)`` encodes ``[S, num_kv_heads, head_dim]`` fp32 tokens in one
    launch: per token and head the scale s = max(1e-8, max|k|)/127
    (ojasx_lut_kv_cache.cpp:29-34) and per group of ``block_dim`` coordinates
    the nearest of the 256 centroids of ``k_codebook``/``v_codebook``
    ([num_kv_heads, 256, block_dim] or one [256, block_dim] for all heads),
    or, with no codebooks, the reference's scalar quantiser.  ``decode(q)``
    runs the paged code-domain attention of ``[num_q_heads, head_dim]``
    queries over the resident tokens.
    """

    def __init__(self, num_kv_heads: int, head_dim: int = 128, block_dim: int = 16,
                 page_size: int = 16, max_resident_pages: int = 2048, sink_pages: int = 2,
                 k_codebook=None, v_codebook=None, device="cuda") -> None:
        torch = _torch()
        if head_dim <= 0 or block_dim <= 0 or head_dim % block_dim:
            raise ValueError("head_dim must be a positive multiple of block_dim")
        if head_dim // block_dim > 32 or block_dim > 32:
            raise ValueError("the decode kernels take head_dim / block_dim <= 32, block_dim <= 32")
        if (k_codebook is None) != (v_codebook is None):
            raise ValueError("give both codebooks or neither")
        self.table = PageTable(page_size, max_resident_pages, sink_pages)
        self.num_kv_heads, self.head_dim, self.block_dim = num_kv_heads, head_dim, block_dim
        self.page_size, self.max_resident_pages, self.sink_pages = (
            page_size, max_resident_pages, sink_pages)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("PagedCodeKVCache runs on the GPU only")
        G = head_dim // block_dim
        self.total_tokens_seen = 0
        self.scalar_codes = k_codebook is None
        if self.scalar_codes:
            # The reference's implicit codebook C[c] = (c - 128) e_0.
            cb = torch.zeros(num_kv_heads, 256, block_dim, dtype=torch.float32)
            cb[:, :, 0] = torch.arange(256, dtype=torch.float32) - 128
            self.k_codebook = cb.to(self.device)
            self.v_codebook = self.k_codebook
        else:
            self.k_codebook = self._codebook(k_codebook)
            self.v_codebook = self._codebook(v_codebook)
        shape = (max_resident_pages, num_kv_heads, page_size)
        self.k_codes = torch.zeros(*shape, G, dtype=torch.uint8, device=self.device)
        self.v_codes = torch.zeros_like(self.k_codes)
        self.k_scales = torch.zeros(shape, dtype=torch.float32, device=self.device)
        self.v_scales = torch.zeros_like(self.k_scales)
        self._bt = torch.zeros(max_resident_pages, dtype=torch.int32, device=self.device)
        self._bt_pages: Optional[List[int]] = None

    def _codebook(self, cb):
        torch = _torch()
        cb = torch.as_tensor(cb, dtype=torch.float32)
        if cb.dim() == 2:
            cb = cb.unsqueeze(0).expand(self.num_kv_heads, -1, -1)
        if tuple(cb.shape) != (self.num_kv_heads, 256, self.block_dim):
            raise ValueError(f"codebook must be [num_kv_heads, 256, {self.block_dim}] or "
                             f"[256, {self.block_dim}], got {tuple(cb.shape)}")
        return cb.to(self.device).contiguous()

    def append(self, k, v) -> None:
        torch = _torch()
        _require_gpu(k, "PagedCodeKVCache.append")
        _require_gpu(v, "PagedCodeKVCache.append")
        if k.dim() == 2:
            k, v = k.unsqueeze(0), v.unsqueeze(0)
        want = (self.num_kv_heads, self.head_dim)
        if k.dim() != 3 or tuple(k.shape[1:]) != want or k.shape != v.shape:
            raise ValueError(f"k and v must be [S, {want[0]}, {want[1]}] of one shape")
        n = k.shape[0]
        self.total_tokens_seen += n
        if n == 0:
            return
        slots = torch.from_numpy(self.table.plan(n)).to(self.device)
        k = k.to(torch.float32).contiguous()
        v = v.to(torch.float32).contiguous()
        cbk = None if self.scalar_codes else _vp(self.k_codebook)
        cbv = None if self.scalar_codes else _vp(self.v_codebook)
        rc = _lib.lib().ojasx_kv_encode_append_device(
            _vp(k), _vp(v), n, self.num_kv_heads, self.head_dim, self.block_dim, cbk, cbv,
            _vp(slots), self.page_size, self.max_resident_pages, _vp(self.k_codes),
            _vp(self.k_scales), _vp(self.v_codes), _vp(self.v_scales), _stream())
        _lib.check(rc, "ojasx_kv_encode_append_device")

    @property
    def seq_len(self) -> int:
        return self.table.seq_len

    resident_tokens = seq_len

    def block_table(self):
        """Device int32 block table of the resident pages, in logical order."""
        torch = _torch()
        pages = self.table.pages
        if self._bt_pages != pages:
            if pages:
                self._bt[:len(pages)].copy_(torch.tensor(pages, dtype=torch.int32))
            self._bt_pages = list(pages)
        return self._bt

    def decode(self, q, scale_factor: float = -1.0, out=None):
        """Attention of q [num_q_heads, head_dim] (fp32) over the resident
        tokens; q head j reads kv head j // (num_q_heads // num_kv_heads).
        ``scale_factor <= 0`` means 1/sqrt(head_dim).  An empty cache gives 0."""
        torch = _torch()
        _require_gpu(q, "PagedCodeKVCache.decode")
        q = q.to(torch.float32).contiguous()
        Hq = q.shape[0]
        if q.dim() != 2 or q.shape[1] != self.head_dim or Hq % self.num_kv_heads:
            raise ValueError("q must be [num_q_heads, head_dim], num_q_heads a multiple of "
                             "num_kv_heads")
        if out is None:
            out = torch.zeros(Hq, self.head_dim, dtype=torch.float32, device=q.device)
        T = self.seq_len
        if T:
            rc = _lib.lib().ojasx_kv_decode_paged_device(
                _vp(q), _vp(self.k_codes), _vp(self.k_scales), _vp(self.v_codes),
                _vp(self.v_scales), _vp(self.k_codebook), _vp(self.v_codebook),
                _vp(self.block_table()), T, self.page_size, Hq, self.num_kv_heads,
                self.head_dim, self.block_dim, float(scale_factor), _vp(out), _stream())
            _lib.check(rc, "ojasx_kv_decode_paged_device")
        return out

    @property
    def storage_bytes(self) -> int:
        """Codes and scales of the resident tokens (K and V)."""
        G = self.head_dim // self.block_dim
        return 2 * self.seq_len * self.num_kv_heads * (G + 4)
