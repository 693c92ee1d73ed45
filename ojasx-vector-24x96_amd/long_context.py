"""Paged KV storage on the GPU, on the kernels of csrc/kv_pages.hip and
csrc/lut_kv.hip.

* ``PagedCompressedKVCache`` mirrors ojasx_24x96/long_context.py:212-279: the
  int8 cache with per-token fp16 scales and sink + sliding-window eviction.
  Names, argument meaning, validation, the page list ``_pages`` of
  ``(qk, sk, qv, sv)`` and ``storage_bytes`` match the reference.  Each page
  gets tensors of its own length, so an evicted page keeps its values for a
  caller that still holds it, as the reference's popped page does; the memory
  of an evicted page nobody holds returns to torch's caching allocator and is
  reused by a later page without a device allocation.
* ``PagedCodeKVCache`` is the code-domain counterpart for decode: per token
  and kv head, 8-bit codes into a 256-centroid codebook (or the reference's
  scalar quantiser, ojasx_lut_kv_cache.cpp:16-65) and an fp32 scale, in the
  page layout [page][kv head][slot][group] that ``decode`` reads through a
  block table.  Tokens fill pages in order; opening a page beyond
  ``max_resident_pages`` evicts the oldest page after the ``sink_pages`` first
  ones (the reference's eviction rule, long_context.py:255-257).

* ``OnlineSoftmaxBlockAttention`` mirrors long_context.py:47-209: exact
  attention over streamed (K, V) tiles with fp64 online-softmax state, on the
  kernels of csrc/attn_stream.hip.  ``forward_stream`` takes any iterable of
  tiles (one device update per tile, tiles moved to the query's device as the
  reference moves them) or a ``PagedCompressedKVCache`` itself, whose int8
  pages are then read in place and dequantised in registers, all pages in
  one update.

Everything runs on the GPU; CPU queries raise.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Iterable, Iterator, List, Optional, Tuple

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
    tags = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.float64: 3}
    if dtype not in tags:
        raise TypeError(f"unsupported KV dtype {dtype}: float32, bfloat16, float16 or float64")
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
        self._layout = None              # (B, H, D, device) of the first append
        self._version = 0                # bumped by every append
        self._tiles = None               # (version, attention tile array, tokens, max page)

    @staticmethod
    def _quantize_int8(t):
        """long_context.py:234-240 on the GPU: t [..., D] float32/bfloat16/
        float16/float64 -> (q int8 [..., D], scale float16 [..., 1])."""
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

    @staticmethod
    def _new_page(B, H, n, D, device):
        torch = _torch()
        qk = torch.empty(B, H, n, D, dtype=torch.int8, device=device)
        sk = torch.empty(B, H, n, 1, dtype=torch.float16, device=device)
        return qk, sk, torch.empty_like(qk), torch.empty_like(sk)

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
        self._version += 1
        key, value = key.contiguous(), value.contiguous()
        for start in range(0, S, self.page_size):
            n = min(start + self.page_size, S) - start
            if len(self._pages) == self.max_resident_pages:
                # Evicting before the append leaves the same pages as the
                # reference's append-then-pop(sink_pages); the popped page's
                # memory can then serve the new page when nobody holds it.
                self._pages.pop(self.sink_pages)
            qk, sk, qv, sv = self._new_page(B, H, n, D, key.device)
            _quantize_into(key[:, :, start:start + n], qk, sk)
            _quantize_into(value[:, :, start:start + n], qv, sv)
            self._pages.append((qk, sk, qv, sv))

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


@dataclass(frozen=True)
class BlockAttentionReport:
    """Telemetry of an online-softmax pass (long_context.py:36-44)."""

    query_tokens: int
    kv_tokens: int
    num_kv_blocks: int
    peak_tile_elements: int
    max_logsumexp: float


def _attn_tag(dtype):
    torch = _torch()
    return {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16,
            torch.float16: _lib.DTYPE_F16, torch.float64: _lib.DTYPE_F64}.get(dtype)


def _float_tile(k, v, keep):
    """AttnTile of float K/V blocks [B, H_kv, S, D] (k and v of one dtype,
    rows contiguous and aligned; otherwise contiguous copies, kept alive in
    ``keep`` until the update is enqueued)."""
    torch = _torch()
    if k.dtype != v.dtype or _attn_tag(k.dtype) is None:
        k, v = k.to(torch.float64), v.to(torch.float64)
    es = k.element_size()
    ak, av = min(16, 8 * es), min(16, 4 * es)

    def fits(t, a):
        return (t.stride(-1) == 1 and t.data_ptr() % a == 0 and
                all((st * es) % ak == 0 for st in t.stride()[:3]) and t.stride(2) >= t.shape[3])

    if not fits(k, ak) or not fits(v, av) or k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    keep.extend((k, v))
    tile = _lib.AttnTile(k.data_ptr(), v.data_ptr(), None, None, k.shape[2],
                         k.stride(0), k.stride(1), k.stride(2), 0, 0, 0)
    return tile, _attn_tag(k.dtype)


class OnlineSoftmaxBlockAttention:
    """Exact attention of queries over streamed (K, V) tiles with fp64
    (m, l, acc) state (long_context.py:47-209): MHA, GQA and MQA, optional
    causal masking.  Constructor arguments, validation and the scale
    1/sqrt(head_dim) follow the reference; the arithmetic runs on the GPU
    (scores and state in fp64, tiles read in their own type)."""

    def __init__(self, num_heads: int, num_kv_heads: Optional[int] = None, head_dim: int = 64,
                 *, q_block_size: int = 128, kv_block_size: int = 256,
                 causal: bool = True) -> None:
        if min(num_heads, head_dim, q_block_size, kv_block_size) <= 0:
            raise ValueError("Attention dimensions and block sizes must be positive")
        self.num_heads = int(num_heads)
        self.num_kv_heads = int(num_kv_heads or num_heads)
        if self.num_heads % self.num_kv_heads != 0:
            raise ValueError(f"num_heads ({self.num_heads}) must be divisible by num_kv_heads "
                             f"({self.num_kv_heads})")
        self.num_queries_per_kv = self.num_heads // self.num_kv_heads
        self.head_dim = int(head_dim)
        self.q_block_size = int(q_block_size)
        self.kv_block_size = int(kv_block_size)
        self.causal = bool(causal)
        self.scale = 1.0 / math.sqrt(self.head_dim)
        # the kernels take head dims in multiples of 8: others run zero-padded
        # to the next one (exact: the added products are fp64 zeros; the
        # scale stays 1/sqrt(head_dim)) and the output is cut back
        self._dpad = -(-self.head_dim // 8) * 8

    def _pad_d(self, t):
        extra = self._dpad - t.shape[-1]
        return t if extra == 0 else _torch().nn.functional.pad(t, (0, extra))

    def _expand_kv_heads(self, tensor):
        """[B, H_kv, S, D] -> [B, H_q, S, D], each kv head repeated for its
        query heads (a view)."""
        if self.num_queries_per_kv == 1:
            return tensor
        B, H_kv, S, D = tensor.shape
        return tensor.unsqueeze(2).expand(B, H_kv, self.num_queries_per_kv, S, D).reshape(
            B, self.num_heads, S, D)

    def _check_query(self, query):
        if query.dim() != 4:
            raise ValueError(f"Expected query [B, H, S_q, D], got {tuple(query.shape)}")
        B, H_q, S_q, D = query.shape
        if H_q != self.num_heads or D != self.head_dim:
            raise ValueError(f"Expected query heads={self.num_heads}, dim={self.head_dim}, "
                             f"got ({H_q}, {D})")
        _require_gpu(query, "OnlineSoftmaxBlockAttention")
        if _attn_tag(query.dtype) is None:
            raise TypeError(f"unsupported query dtype {query.dtype}: float32, bfloat16, "
                            "float16 or float64")

    def _init(self, query):
        torch = _torch()
        B, H_q, S_q, D = query.shape
        rows = B * H_q * S_q
        state = torch.empty(rows, 2 * D + 2, dtype=torch.float64, device=query.device)
        q = query.contiguous()
        rc = _lib.lib().ojasx_attention_stream_init_device(_vp(state), _vp(q), _attn_tag(q.dtype),
                                                          rows, D, _stream())
        _lib.check(rc, "ojasx_attention_stream_init_device")
        return state

    def _page_tiles(self, cache, query):
        """The cache's resident pages as int8 attention tiles, rebuilt only
        after an append: (tile array, resident tokens, longest page)."""
        if cache._tiles is not None and cache._tiles[0] == cache._version:
            return cache._tiles[1:]
        tiles = []
        for qk, sk, qv, sv in cache._pages:
            if qk.device != query.device:
                raise ValueError("the cache's pages live on another device than the query")
            self._check_block(qk, query.shape[0], "key")
            if qk.shape[2]:
                tiles.append(_lib.AttnTile(qk.data_ptr(), qv.data_ptr(), sk.data_ptr(),
                                           sv.data_ptr(), qk.shape[2], qk.stride(0), qk.stride(1),
                                           qk.stride(2), sk.stride(0), sk.stride(1), sk.stride(2)))
        arr = (_lib.AttnTile * len(tiles))(*tiles)
        cache._tiles = (cache._version, arr, sum(t.n_tokens for t in tiles),
                        max((t.n_tokens for t in tiles), default=0))
        return cache._tiles[1:]

    def _update(self, state, query, tiles, kv_tag, query_start_pos, kv_offset):
        B, H_q, S_q, D = query.shape
        arr = tiles if isinstance(tiles, ctypes.Array) else (_lib.AttnTile * len(tiles))(*tiles)
        rc = _lib.lib().ojasx_attention_stream_update_device(
            _vp(state), B, H_q, self.num_kv_heads, S_q, D, arr, len(tiles), kv_tag,
            int(self.causal), int(query_start_pos), int(kv_offset), float(self.scale), _stream())
        _lib.check(rc, "ojasx_attention_stream_update_device")

    def _finalize(self, state, query, lse=None):
        torch = _torch()
        out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
        rc = _lib.lib().ojasx_attention_stream_finalize_device(
            _vp(state), state.shape[0], query.shape[3], _vp(out), _attn_tag(query.dtype),
            _vp(lse) if lse is not None else None, _stream())
        _lib.check(rc, "ojasx_attention_stream_finalize_device")
        return out

    def _check_block(self, t, B, name):
        if t.dim() != 4 or t.shape[0] != B or t.shape[1] != self.num_kv_heads or \
                t.shape[3] != self.head_dim:
            raise ValueError(f"Expected {name} block [B={B}, H_kv={self.num_kv_heads}, S, "
                             f"D={self.head_dim}], got {tuple(t.shape)}")

    def forward_stream(self, query, kv_stream, *, query_start_pos: int = 0):
        """Attention of ``query`` [B, H_q, S_q, D] over a stream of
        ``(K_block, V_block)`` tiles [B, H_kv, S_k, D] (long_context.py:92-176),
        or over every resident page of a ``PagedCompressedKVCache`` passed
        as the stream.  Returns ``(out, BlockAttentionReport)``; ``out`` has
        the query's dtype."""
        torch = _torch()
        self._check_query(query)
        B, H_q, S_q, D = query.shape
        qp = self._pad_d(query)
        state = self._init(qp)
        kv_offset = num_blocks = peak = 0
        if isinstance(kv_stream, PagedCompressedKVCache) and kv_stream._pages and \
                kv_stream._pages[0][0].shape[3] % 16 == 0:
            self._check_block(kv_stream._pages[0][0], B, "key")
            arr, kv_offset, max_n = self._page_tiles(kv_stream, query)
            num_blocks = len(arr)
            peak = B * H_q * S_q * max_n
            self._update(state, qp, arr, _lib.DTYPE_INT8, query_start_pos, 0)
        else:
            if isinstance(kv_stream, PagedCompressedKVCache):
                kv_stream = kv_stream.iter_dequantized_pages()   # head_dim not a multiple of 16

            for k_blk, v_blk in kv_stream:
                k_blk = k_blk.to(device=query.device)
                v_blk = v_blk.to(device=query.device)
                self._check_block(k_blk, B, "key")
                self._check_block(v_blk, B, "value")
                if k_blk.shape[2] != v_blk.shape[2]:
                    raise ValueError("key and value blocks differ in length")
                S_k = k_blk.shape[2]
                if S_k == 0:
                    continue
                keep = []
                tile, tag = _float_tile(self._pad_d(k_blk), self._pad_d(v_blk), keep)
                self._update(state, qp, [tile], tag, query_start_pos, kv_offset)
                num_blocks += 1
                peak = max(peak, B * H_q * S_q * S_k)
                kv_offset += S_k
        lse = torch.empty(state.shape[0], dtype=torch.float64, device=query.device)
        out = self._finalize(state, qp, lse)
        if qp is not query:
            out = out[..., :D].contiguous()
        # the rows' log-sum-exps copied out and reduced on the host: one
        # synchronising copy, no reduction kernel
        max_lse = float(lse.cpu().max()) if kv_offset > 0 else 0.0
        return out, BlockAttentionReport(query_tokens=S_q, kv_tokens=kv_offset,
                                         num_kv_blocks=num_blocks, peak_tile_elements=peak,
                                         max_logsumexp=max_lse)

    def forward(self, query, key, value, *, query_start_pos: int = 0):
        """Tiled exact attention of ``query`` over ``key`` / ``value``
        [B, H_kv, S_k, D] (long_context.py:178-209): query blocks of
        q_block_size, each over the kv blocks of kv_block_size its causal
        horizon reaches, all of a query block's kv blocks in one update."""
        torch = _torch()
        self._check_query(query)
        B, H_q, S_q, D = query.shape
        key = key.to(device=query.device)
        value = value.to(device=query.device)
        self._check_block(key, B, "key")
        self._check_block(value, B, "value")
        key, value, qp = self._pad_d(key), self._pad_d(value), self._pad_d(query)
        S_k = key.shape[2]
        outs = []
        for q_start in range(0, S_q, self.q_block_size):
            q_stop = min(q_start + self.q_block_size, S_q)
            q_chunk = qp[:, :, q_start:q_stop, :]
            eff_k = min(S_k, query_start_pos + q_stop) if self.causal else S_k
            state = self._init(q_chunk)
            keep, tiles, tag = [], [], None
            for k_start in range(0, max(eff_k, 0), self.kv_block_size):
                k_stop = min(k_start + self.kv_block_size, eff_k)
                tile, tag = _float_tile(key[:, :, k_start:k_stop, :],
                                        value[:, :, k_start:k_stop, :], keep)
                tiles.append(tile)
            if tiles:
                self._update(state, q_chunk, tiles, tag, query_start_pos + q_start, 0)
            outs.append(self._finalize(state, q_chunk))
        out = torch.cat(outs, dim=2)
        return out if qp is query else out[..., :D].contiguous()

    __call__ = forward


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
