"""Greedy batch-1 decoder on the LUT engine: a Qwen3-4B-shaped stack (RMSNorm,
per-head q/k RMSNorm, RoPE, GQA attention over the paged code KV cache,
SwiGLU MLP) whose every linear is a split-manifold LUT linear with CSR
outliers, run by the HIP decoder of csrc/decoder.hip (C-ABI
``ojasx_create_decoder`` and friends).

``LUTDecoder`` holds the device decoder and keeps the linear handles it
references alive.  ``synthetic_decoder`` builds one with seeded random weights
and a random prefilled code context: the reference's 4B-shaped benchmark
configuration (hidden 2560, 36 layers, 32 q / 8 kv heads, head dim 128, MLP
9728, 4096-token 8-bit KV context) by default.  All tensors live on the GPU;
there is no CPU path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from . import _lib
from .native import NativeSplitManifoldLinear


def _torch():
    import torch
    return torch


def _vp(t):
    return ctypes.c_void_p(t.data_ptr())


def _dev_f32(a, device):
    torch = _torch()
    t = torch.as_tensor(a, dtype=torch.float32)
    return t.to(device).contiguous()


@dataclass
class DecoderConfig:
    hidden: int = 2560
    layers: int = 36
    q_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 9728
    vocab: int = 151936
    max_context: int = 4096 + 128
    page_size: int = 16
    max_steps: int = 128
    rms_eps: float = 1e-6
    rope_theta: float = 1e6


class LUTDecoder:
    """Device decoder.  Linears are ``NativeSplitManifoldLinear`` objects (or
    raw handles) with block_dim 16: qkv hidden -> (q + 2 kv heads) * 128 (q
    rows, then k, then v), o -> hidden, gate_up -> 2 * intermediate (gate rows,
    then up rows), down -> hidden, lm_head hidden -> vocab."""

    def __init__(self, cfg: DecoderConfig = DecoderConfig(), device="cuda"):
        self.cfg = cfg
        self.device = device
        self._keep: List[object] = []
        h = _lib.lib().ojasx_create_decoder(cfg.hidden, cfg.layers, cfg.q_heads, cfg.kv_heads,
                                            cfg.head_dim, cfg.intermediate, cfg.vocab,
                                            cfg.max_context, cfg.page_size, cfg.max_steps,
                                            cfg.rms_eps, cfg.rope_theta)
        if not h:
            raise RuntimeError("ojasx_create_decoder failed: "
                               + _lib.lib().ojasx_get_last_error().decode(errors="replace"))
        self._destroy = _lib.lib().ojasx_destroy_decoder
        self._h = h

    @staticmethod
    def _handle(lin):
        return lin.handle if isinstance(lin, NativeSplitManifoldLinear) else lin

    def set_layer(self, layer, qkv, o, gate_up, down, input_norm, post_norm, q_norm, k_norm,
                  k_codebook, v_codebook):
        t = [_dev_f32(a, self.device) for a in (input_norm, post_norm, q_norm, k_norm,
                                                 k_codebook, v_codebook)]
        rc = _lib.lib().ojasx_decoder_set_layer(
            self._h, layer, self._handle(qkv), self._handle(o), self._handle(gate_up),
            self._handle(down), *[_vp(a) for a in t])
        _lib.check(rc, "ojasx_decoder_set_layer")
        self._keep += [qkv, o, gate_up, down]

    def set_head(self, lm_head, final_norm, embedding):
        fn = _dev_f32(final_norm, self.device)
        emb = _dev_f32(embedding, self.device)
        rc = _lib.lib().ojasx_decoder_set_head(self._h, self._handle(lm_head), _vp(fn), _vp(emb))
        _lib.check(rc, "ojasx_decoder_set_head")
        self._keep.append(lm_head)

    def set_context(self, layer, k_codes, k_scales, v_codes, v_scales, num_tokens):
        """Prefilled context of one layer in the paged layout
        [pages][kv_heads][page_size][8] / [pages][kv_heads][page_size]."""
        torch = _torch()
        kc = torch.as_tensor(k_codes, dtype=torch.uint8).to(self.device).contiguous()
        vc = torch.as_tensor(v_codes, dtype=torch.uint8).to(self.device).contiguous()
        ks = _dev_f32(k_scales, self.device)
        vs = _dev_f32(v_scales, self.device)
        rc = _lib.lib().ojasx_decoder_set_context(self._h, layer, _vp(kc), _vp(ks), _vp(vc),
                                                  _vp(vs), num_tokens)
        _lib.check(rc, "ojasx_decoder_set_context")

    def reset(self, position: int):
        _lib.check(_lib.lib().ojasx_decoder_reset(self._h, position), "ojasx_decoder_reset")

    def generate(self, first_token: int, num_tokens: int, use_graph: bool = True,
                 return_logits: bool = False):
        """Greedy tokens after ``first_token`` (and the last step's logits)."""
        toks = np.zeros(num_tokens, np.int32)
        logits = np.zeros(self.cfg.vocab, np.float32) if return_logits else None
        rc = _lib.lib().ojasx_decoder_generate(
            self._h, int(first_token), int(num_tokens), 1 if use_graph else 0,
            toks.ctypes.data_as(ctypes.c_void_p),
            logits.ctypes.data_as(ctypes.c_void_p) if logits is not None else None)
        _lib.check(rc, "ojasx_decoder_generate")
        return (toks, logits) if return_logits else toks

    def read_kv(self, layer: int, first_token: int, num_tokens: int):
        c = self.cfg
        pages = (num_tokens + c.page_size - 1) // c.page_size
        shape = (pages, c.kv_heads, c.page_size)
        kc = np.zeros(shape + (c.head_dim // 16,), np.uint8)
        vc = np.zeros_like(kc)
        ks = np.zeros(shape, np.float32)
        vs = np.zeros_like(ks)
        p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        rc = _lib.lib().ojasx_decoder_read_kv(self._h, layer, first_token, num_tokens, p(kc), p(ks),
                                              p(vc), p(vs))
        _lib.check(rc, "ojasx_decoder_read_kv")
        return kc, ks, vc, vs

    def close(self):
        destroy = getattr(self, "_destroy", None)
        if getattr(self, "_h", None) and destroy is not None:
            destroy(self._h)
            self._h = None
        self._keep = []

    def __del__(self):
        # close() calls the destroy entry point bound at creation: at
        # interpreter exit the module's globals may already be gone
        self.close()


def _linear(r, M, K, sigma, density, sigma_out, keep_dense: bool):
    """A seeded LUT linear: codebook ~ N(0, sigma), uniform codes, unit scales,
    CSR outliers at `density` with |v| ~ U[15, 36] * sigma_out, random sign."""
    from .synthetic import csr_outliers
    cb = r.normal(0.0, sigma, size=(256, 16)).astype(np.float32)
    codes = r.integers(0, 256, size=(M, K // 16), dtype=np.uint8)
    csr = csr_outliers(r, M, K, density, sigma_out)
    lin = NativeSplitManifoldLinear(K, M, 16, 256)
    lin.initialize_weights(cb, codes, np.ones(M, np.float32))
    lin.set_outliers(*csr)
    w = dict(codebook=cb, codes=codes, csr=csr) if keep_dense else None
    return lin, w


def synthetic_decoder(cfg: DecoderConfig = DecoderConfig(), context: int = 4096, seed: int = 0,
                      device="cuda", keep_weights: bool = False, density: float = 0.0038):
    """LUTDecoder with seeded random weights and a random prefilled context of
    ``context`` tokens in every layer; returns (decoder, weights) where weights
    holds the host arrays when ``keep_weights`` (for checking), else None.

    Distributions: linear codebooks ~ N(0, 0.02) with CSR outliers of
    |v| ~ U[15, 36] * 0.02 at ``density``; norm weights ~ U[0.8, 1.2]; KV
    codebooks ~ N(0, 40) per kv head (the encoder works on k / s with
    |k / s| <= 127); context codes uniform with scales ~ U[0.5, 1.5] * 3 / 127;
    embedding rows ~ N(0, 1)."""
    torch = _torch()
    c = cfg
    r = np.random.Generator(np.random.PCG64(seed))
    dec = LUTDecoder(c, device)
    qd, kvd = c.q_heads * c.head_dim, c.kv_heads * c.head_dim
    pages = (context + c.page_size - 1) // c.page_size
    weights: Optional[Dict[str, object]] = {"layers": []} if keep_weights else None
    for layer in range(c.layers):
        qkv, wq = _linear(r, qd + 2 * kvd, c.hidden, 0.02, density, 0.02, keep_weights)
        o, wo = _linear(r, c.hidden, qd, 0.02, density, 0.02, keep_weights)
        gu, wg = _linear(r, 2 * c.intermediate, c.hidden, 0.02, density, 0.02, keep_weights)
        dn, wd = _linear(r, c.hidden, c.intermediate, 0.02, density, 0.02, keep_weights)
        norms = [r.uniform(0.8, 1.2, size=n).astype(np.float32)
                 for n in (c.hidden, c.hidden, c.head_dim, c.head_dim)]
        kcb = r.normal(0.0, 40.0, size=(c.kv_heads, 256, 16)).astype(np.float32)
        vcb = r.normal(0.0, 40.0, size=(c.kv_heads, 256, 16)).astype(np.float32)
        dec.set_layer(layer, qkv, o, gu, dn, *norms, kcb, vcb)
        kc = r.integers(0, 256, size=(pages, c.kv_heads, c.page_size, c.head_dim // 16),
                        dtype=np.uint8)
        vc = r.integers(0, 256, size=kc.shape, dtype=np.uint8)
        ks = (r.uniform(0.5, 1.5, size=kc.shape[:3]) * 3.0 / 127.0).astype(np.float32)
        vs = (r.uniform(0.5, 1.5, size=kc.shape[:3]) * 3.0 / 127.0).astype(np.float32)
        if context:
            dec.set_context(layer, kc, ks, vc, vs, context)
        if keep_weights:
            weights["layers"].append(dict(qkv=wq, o=wo, gate_up=wg, down=wd, input_norm=norms[0],
                                          post_norm=norms[1], q_norm=norms[2], k_norm=norms[3],
                                          k_codebook=kcb, v_codebook=vcb, k_codes=kc, k_scales=ks,
                                          v_codes=vc, v_scales=vs))
    lm, wl = _linear(r, c.vocab, c.hidden, 0.02, density, 0.02, keep_weights)
    final_norm = r.uniform(0.8, 1.2, size=c.hidden).astype(np.float32)
    g = torch.Generator(device=device).manual_seed(seed)
    emb = torch.randn(c.vocab, c.hidden, generator=g, device=device, dtype=torch.float32)
    dec.set_head(lm, final_norm, emb)
    dec.reset(context)
    if keep_weights:
        weights.update(lm_head=wl, final_norm=final_norm, embedding=emb.cpu().numpy())
    return dec, weights
