"""CPU oracle for the fused-MoE forward (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
import this module, and only as the checker / the timed CPU baseline.  The product
(``flash-infer-bench-starter-kit_amd/``) never imports it.

Two layers:

* ``oracle/moe_oracle.c`` (ctypes, built by ``oracle/Makefile``): canonical sigmoid,
  routing, dispatch/permutation, e4m3 decode -- integer/index work that must be
  bit-exact.
* this file: the floating-point expert path restated in torch-CPU fp32, following
  ``solution/cuda/moe.cu:137-240`` of the reference:

  - dequant ``A = e4m3(hs) * hs_scale[h//128, t]`` (moe.cu:52-64, 97-112),
    ``W = e4m3(w) * scale[e, r//128, c//128]`` (moe.cu:73-91, 114-131);
  - per local expert ascending, tokens ascending (moe.cu:212-222):
    ``G1 = A_e @ W13^T``, ``C = silu(G1[:, I:]) * G1[:, :I]``, ``O = C @ W2^T``
    (moe.cu:226-231);
  - ``acc[t] += O * w`` in fp32 (moe.cu:233-235), ``out = bf16(acc)`` (moe.cu:239).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence

import numpy as np
import torch

H, I, N1, E_GLOBAL, E_LOCAL, TOP_K = 7168, 2048, 4096, 256, 32, 8
N_GROUP, GROUP_SIZE, TOPK_GROUP, BLK = 8, 32, 4, 128

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libmoe_oracle.so")
_lib = None


def build() -> str:
    """Compile ``moe_oracle.c`` with ``oracle/Makefile``; returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        L.moe_oracle_sigmoid.restype = ctypes.c_float
        L.moe_oracle_sigmoid.argtypes = [ctypes.c_float]
        L.moe_oracle_exp64.restype = ctypes.c_double
        L.moe_oracle_exp64.argtypes = [ctypes.c_double]
        L.moe_oracle_e4m3_table.restype = None
        L.moe_oracle_e4m3_table.argtypes = [P]
        L.moe_oracle_route.restype = None
        L.moe_oracle_route.argtypes = [P, P, ctypes.c_int32, ctypes.c_double, P, P]
        L.moe_oracle_route_token.restype = None
        L.moe_oracle_route_token.argtypes = [P, P, ctypes.c_double, P, P, P, P, P, P]
        L.moe_oracle_set_mutation.restype = None
        L.moe_oracle_set_mutation.argtypes = [ctypes.c_int]
        L.moe_oracle_dispatch.restype = ctypes.c_int32
        L.moe_oracle_dispatch.argtypes = [P, P, ctypes.c_int32, ctypes.c_int64,
                                          ctypes.c_int32, P, P, P, P, P]
        _lib = L
    return _lib


def set_mutation(m: int) -> None:
    """Plant a known mistake in the C restatement (0 = none); tests only."""
    lib().moe_oracle_set_mutation(int(m))


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _np(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu()
        if x.dtype == torch.bfloat16:
            x = x.view(torch.int16)
        if x.dtype == torch.float8_e4m3fn:
            x = x.view(torch.uint8)
        return np.ascontiguousarray(x.numpy())
    return np.ascontiguousarray(x)


# --------------------------------------------------------------------------- #
# bit-exact layer (C)                                                          #
# --------------------------------------------------------------------------- #

def sigmoid(x: np.ndarray) -> np.ndarray:
    """Canonical fp32 sigmoid (binary64 evaluation, one rounding)."""
    f = lib().moe_oracle_sigmoid
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([f(float(v)) for v in flat], dtype=np.float32).reshape(np.shape(x))


def e4m3_table() -> np.ndarray:
    out = np.zeros(256, dtype=np.float32)
    lib().moe_oracle_e4m3_table(_ptr(out))
    return out


def route(logits, bias_bf16, factor: float):
    """DeepSeek-V3 no-aux routing -> (ids int32 [T,8], w fp32 [T,8]).

    moe.cu:178-206 with the lower-index tie rule of kernel.cu:84-178."""
    lg = _np(logits).astype(np.float32, copy=False)
    lg = np.ascontiguousarray(lg)
    b = _np(bias_bf16).view(np.uint16)
    T = lg.shape[0]
    ids = np.zeros((T, TOP_K), dtype=np.int32)
    w = np.zeros((T, TOP_K), dtype=np.float32)
    if T:
        lib().moe_oracle_route(_ptr(lg), _ptr(b), T, float(factor), _ptr(ids), _ptr(w))
    return ids, w


def route_token_debug(logit_row, bias_bf16, factor: float):
    """One token's routing with intermediate s, s+bias, group scores, kept groups."""
    lg = np.ascontiguousarray(_np(logit_row).astype(np.float32))
    b = _np(bias_bf16).view(np.uint16)
    ids = np.zeros(TOP_K, np.int32)
    w = np.zeros(TOP_K, np.float32)
    s = np.zeros(E_GLOBAL, np.float32)
    sb = np.zeros(E_GLOBAL, np.float32)
    gs = np.zeros(N_GROUP, np.float32)
    keep = np.zeros(1, np.int32)
    lib().moe_oracle_route_token(_ptr(lg), _ptr(b), float(factor), _ptr(ids), _ptr(w),
                                 _ptr(s), _ptr(sb), _ptr(gs), _ptr(keep))
    return dict(ids=ids, w=w, s=s, sb=sb, gscore=gs, keep=int(keep[0]))


def dispatch(ids, w, offset: int, tile_m: int = 64):
    """Canonical (expert asc, token asc) permutation + row tiles.

    Returns dict(exp_off[33], sorted_tok[N_a], sorted_w[N_a], inv[T,8], tiles[nt,4])."""
    ids = np.ascontiguousarray(_np(ids).astype(np.int32))
    w = np.ascontiguousarray(_np(w).astype(np.float32))
    T = ids.shape[0]
    exp_off = np.zeros(E_LOCAL + 1, np.int32)
    stok = np.zeros(max(1, T * TOP_K), np.int32)
    sw = np.zeros(max(1, T * TOP_K), np.float32)
    inv = np.zeros((T, TOP_K), np.int32)
    mt = (T * TOP_K + tile_m - 1) // tile_m + E_LOCAL
    tiles = np.zeros((mt, 4), np.int32)
    nt = lib().moe_oracle_dispatch(_ptr(ids), _ptr(w), T, int(offset), tile_m,
                                   _ptr(exp_off), _ptr(stok), _ptr(sw),
                                   _ptr(inv), _ptr(tiles))
    na = int(exp_off[E_LOCAL])
    return dict(exp_off=exp_off, sorted_tok=stok[:na].copy(), sorted_w=sw[:na].copy(),
                inv=inv, tiles=tiles[:nt].copy())


# --------------------------------------------------------------------------- #
# fp32 expert path (torch CPU)                                                 #
# --------------------------------------------------------------------------- #

def _f8(x) -> torch.Tensor:
    """fp32 decode of an e4m3fn tensor (moe.cu:24-42)."""
    x = x.detach().cpu()
    if x.dtype == torch.uint8:
        x = x.view(torch.float8_e4m3fn)
    return x.to(torch.float32)


def dequant_weight(w_e, scale_e) -> torch.Tensor:
    """``W[r, c] = e4m3(w[r, c]) * scale[r//128, c//128]`` for one expert (moe.cu:73-91)."""
    wf = _f8(w_e)
    s = scale_e.detach().cpu().to(torch.float32)
    s = s.repeat_interleave(BLK, 0).repeat_interleave(BLK, 1)
    return wf * s


def dequant_hidden(hs, hs_scale, tokens: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``A[t, h] = e4m3(hs[t, h]) * hs_scale[h//128, t]`` (moe.cu:52-64)."""
    hs = hs.detach().cpu()
    sc = hs_scale.detach().cpu().to(torch.float32)
    if tokens is not None:
        hs = hs[tokens]
        sc = sc[:, tokens]
    a = _f8(hs)
    return a * sc.t().repeat_interleave(BLK, 1)


def silu(x: torch.Tensor) -> torch.Tensor:
    return x * torch.sigmoid(x)


def hilo_split(C: torch.Tensor):
    """The fp8 hi/lo form of the SwiGLU rows used between the prefill GEMMs (the
    build's own format; the reference re-quantises C to one e4m3 per element with a
    per-128 scale instead, kernel.cu:1086-1145).

    Per row and 128-column block: ``s = amax/448`` (1 if the block is all zero),
    ``hi = e4m3(clamp(c * (448/amax)))``, ``lo = e4m3(clamp((c - hi*s) * 16*448/amax))``
    with ``c - hi*s`` rounded once (an fma).  Returns (hi uint8 [R,2048],
    lo uint8 [R,2048], s fp32 [R,16])."""
    C = C.detach().to(torch.float32)
    R = C.shape[0]
    b = C.reshape(R, I // BLK, BLK)
    amax = b.abs().amax(dim=2, keepdim=True)
    nz = amax > 0
    s = torch.where(nz, amax / 448.0, torch.ones_like(amax))
    inv = torch.where(nz, 448.0 / amax, torch.ones_like(amax))
    hi = (b * inv).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    res = (b.double() - hi.to(torch.float64) * s.double()).to(torch.float32)
    lo = (res * (inv * 16.0)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return (hi.view(torch.uint8).reshape(R, I), lo.view(torch.uint8).reshape(R, I),
            s.reshape(R, I // BLK))


def hilo_join(hi: torch.Tensor, lo: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """``s * (e4m3(hi) + e4m3(lo) / 16)`` per 128-column block, fp32 [R, 2048]."""
    R = hi.shape[0]
    h = hi.view(torch.float8_e4m3fn).to(torch.float32).reshape(R, I // BLK, BLK)
    l = lo.view(torch.float8_e4m3fn).to(torch.float32).reshape(R, I // BLK, BLK)
    return ((h + l / 16.0) * s.reshape(R, I // BLK, 1)).reshape(R, I)


def swiglu_rows(hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
                le: int, tokens: Sequence[int]) -> torch.Tensor:
    """fp32 C rows ``silu(G1[:, I:]) * G1[:, :I]`` of local expert ``le`` for ``tokens``
    (moe.cu:226-229)."""
    A = dequant_hidden(hidden_states, hidden_states_scale, torch.as_tensor(list(tokens), dtype=torch.int64))
    W13 = dequant_weight(gemm1_weights[le], gemm1_weights_scale[le])
    G1 = A @ W13.t()
    return silu(G1[:, I:]) * G1[:, :I]


def expert_forward(hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
                   gemm2_weights, gemm2_weights_scale, ids, w, offset: int,
                   tokens: Optional[Sequence[int]] = None,
                   intermediate_dtype: torch.dtype = torch.float32,
                   rows_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """fp32 accumulator ``acc`` [len(tokens) or T, H] before the bf16 cast.

    ``tokens`` restricts the computation to a subset of tokens (each output row
    depends only on its own token, so a subset is an exact restatement for those
    rows).  ``intermediate_dtype`` rounds C = silu(x2)*x1 before GEMM2 (fp32 = the
    reference; bf16, fp16, float8 or "hilo" (``hilo_split``) study the precision of
    the forms the GPU path keeps C in); ``rows_dtype`` likewise rounds each expert's
    output row O before the weighted sum (fp32 = the reference)."""
    ids = torch.as_tensor(_np(ids)).to(torch.int64)
    wt = torch.as_tensor(_np(w)).to(torch.float32)
    T = ids.shape[0]
    tok = torch.arange(T) if tokens is None else torch.as_tensor(list(tokens), dtype=torch.int64)
    sub_ids = ids[tok]
    sub_w = wt[tok]
    acc = torch.zeros(len(tok), H, dtype=torch.float32)
    if len(tok) == 0:
        return acc
    A = dequant_hidden(hidden_states, hidden_states_scale, tok)
    for le in range(E_LOCAL):
        ge = int(offset) + le
        if ge < 0 or ge >= E_GLOBAL:
            continue
        hit = (sub_ids == ge)
        sel = hit.any(dim=1).nonzero().squeeze(1)
        if sel.numel() == 0:
            continue
        W13 = dequant_weight(gemm1_weights[le], gemm1_weights_scale[le])
        W2 = dequant_weight(gemm2_weights[le], gemm2_weights_scale[le])
        G1 = A[sel] @ W13.t()
        C = silu(G1[:, I:]) * G1[:, :I]
        if intermediate_dtype == "hilo":
            C = hilo_join(*hilo_split(C))
        elif intermediate_dtype != torch.float32:
            C = C.to(intermediate_dtype).to(torch.float32)
        O = C @ W2.t()
        if rows_dtype != torch.float32:
            O = O.to(rows_dtype).to(torch.float32)
        wk = (sub_w[sel] * hit[sel].to(torch.float32)).sum(dim=1, keepdim=True)
        acc.index_add_(0, sel, O * wk)
    return acc


def forward(routing_logits, routing_bias, hidden_states, hidden_states_scale,
            gemm1_weights, gemm1_weights_scale, gemm2_weights, gemm2_weights_scale,
            local_expert_offset: int, routed_scaling_factor: float,
            tokens: Optional[Sequence[int]] = None):
    """Whole operator on the CPU: returns (bf16 out, fp32 acc, ids, w)."""
    ids, w = route(routing_logits, routing_bias, routed_scaling_factor)
    acc = expert_forward(hidden_states, hidden_states_scale, gemm1_weights,
                         gemm1_weights_scale, gemm2_weights, gemm2_weights_scale,
                         ids, w, local_expert_offset, tokens)
    return acc.to(torch.bfloat16), acc, ids, w


# --------------------------------------------------------------------------- #
# activation quantizer, the step before the operator (kernel.cu:998-1062)     #
# --------------------------------------------------------------------------- #

def e4m3_encode_rne(v, _ties: str = "even") -> np.ndarray:
    """fp32 -> e4m3fn bytes, round to nearest, ties to even, for |v| <= 448.

    Written from the OCP FP8 E4M3 definition on the decode table of moe_oracle.c (the
    127 non-negative finite codes 0x00..0x7E have increasing magnitudes): the nearest
    code, on a tie the one with an even mantissa (code & 1 == 0); the sign bit copied,
    so -0.0 gives 0x80.  Values above 448 saturate to 448 (callers clamp first).
    ``_ties="away"`` is a planted mistake for the pin tests only."""
    v = np.asarray(v, dtype=np.float32)
    tab = e4m3_table()[:127].astype(np.float64)
    a = np.abs(v.astype(np.float64)).ravel()
    hi = np.clip(np.searchsorted(tab, a, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    dlo = a - tab[lo]
    dhi = tab[hi] - a
    if _ties == "even":
        tie_hi = (hi % 2) == 0
    elif _ties == "away":
        tie_hi = np.ones_like(hi, dtype=bool)
    else:
        raise ValueError(_ties)
    code = np.where((dhi < dlo) | ((dhi == dlo) & tie_hi), hi, lo).astype(np.uint8)
    code |= (np.signbit(v).ravel().astype(np.uint8) << 7)
    return code.reshape(v.shape)


def quantize_fp8_blockwise(x, _block_amax: bool = True):
    """Blockwise FP8 quantizer (solution/python/kernel.cu:998-1062) in fp32 numpy.

    ``x`` [rows, cols] (float32, or bfloat16 as a torch tensor; widened exactly).  Per
    row and 128-column block: ``absmax`` with fmaxf semantics (NaN ignored,
    kernel.cu:1020-1024), ``scale = absmax / 448`` or 1 for an all-zero block
    (kernel.cu:1037), ``inv = 1 / scale`` (1038), ``q = e4m3(fminf(fmaxf(x * inv,
    -448), 448))`` round to nearest even (999-1002, 1048-1050).  Returns (q uint8
    [rows, cols], scales fp32 [cols / 128, rows]) (column-major scales, 1041-1044).
    ``_block_amax=False`` (one absmax per row) is a planted mistake for the pin tests."""
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu().to(torch.float32).numpy()
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    nb = cols // BLK
    b = x.reshape(rows, nb, BLK)
    amax = np.fmax.reduce(np.abs(b), axis=2, initial=np.float32(0.0)).astype(np.float32)
    if not _block_amax:
        amax = np.repeat(np.fmax.reduce(amax, axis=1, initial=np.float32(0.0))[:, None], nb, axis=1)
    scale = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    y = (b * inv[:, :, None]).astype(np.float32)
    y = np.fmin(np.fmax(y, np.float32(-448.0)), np.float32(448.0))
    q = e4m3_encode_rne(y).reshape(rows, cols)
    return q, np.ascontiguousarray(scale.T)


# --------------------------------------------------------------------------- #
# CPU baseline: the reference's own CPU-shaped path (moe.cu:137-240)           #
# --------------------------------------------------------------------------- #

def reference_cpu_forward(routing_logits, routing_bias, hidden_states, hidden_states_scale,
                          gemm1_weights, gemm1_weights_scale, gemm2_weights,
                          gemm2_weights_scale, local_expert_offset: int,
                          routed_scaling_factor: float, output: torch.Tensor) -> None:
    """The moe.cu control flow on host tensors: dequant everything to fp32
    (moe.cu:164-176), route (178-206), per-expert loop (208-236), bf16 copy (239).

    Used as the timed CPU baseline; ``output`` is written in place (DPS)."""
    E = gemm1_weights.shape[0]
    A = dequant_hidden(hidden_states, hidden_states_scale)

    def deq(w, s):  # [E, R, C] e4m3 * [E, R/128, C/128] broadcast over 128x128 blocks
        e, r, c = w.shape
        wf = _f8(w).view(e, r // BLK, BLK, c // BLK, BLK)
        return (wf * s.float().view(e, r // BLK, 1, c // BLK, 1)).view(e, r, c)

    W13 = deq(gemm1_weights, gemm1_weights_scale)
    W2 = deq(gemm2_weights, gemm2_weights_scale)
    ids, w = route(routing_logits, routing_bias, routed_scaling_factor)
    ids = torch.from_numpy(ids).to(torch.int64)
    wt = torch.from_numpy(w)
    acc = torch.zeros(A.shape[0], H, dtype=torch.float32)
    for le in range(E):
        ge = int(local_expert_offset) + le
        if ge < 0 or ge >= E_GLOBAL:
            continue
        hit = ids == ge
        sel = hit.any(dim=1).nonzero().squeeze(1)
        if sel.numel() == 0:
            continue
        G1 = A[sel] @ W13[le].t()
        C = silu(G1[:, I:]) * G1[:, :I]
        O = C @ W2[le].t()
        wk = (wt[sel] * hit[sel].to(torch.float32)).sum(dim=1, keepdim=True)
        acc.index_add_(0, sel, O * wk)
    output.copy_(acc.to(torch.bfloat16))


