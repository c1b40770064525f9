"""Quantized weight formats and their upload (src/weights.rs counterparts).

QuantConfig mirrors src/weights.rs:154-167. GptqWeight holds one GPTQ linear
on the device in the reference layout (qweight u32[K/8, N], scales f16[G, N])
plus what the reference drops at load (src/weights.rs:372-374): qzeros and
g_idx. An act-order g_idx is resolved at upload by st_gptq_i4_act_order
(rows sorted by group, values unchanged). Int8Weight is the INT8
per-channel format (no reference counterpart).
"""
from __future__ import annotations

import json
from dataclasses import dataclass

import numpy as np

from ._lib import ST_FLAG_TILED, ST_FLAG_ZEROS_PLUS_ONE, call, lib


@dataclass
class QuantConfig:
    """quantize_config.json (src/weights.rs:154-167); the reference reads
    only group_size (src/model.rs:366)."""

    bits: int = 4
    group_size: int = 128
    quant_method: str = "gptq"
    sym: bool = True

    @classmethod
    def from_dict(cls, d: dict) -> "QuantConfig":
        return cls(
            bits=int(d.get("bits", 4)),
            group_size=int(d.get("group_size", 128)),
            quant_method=str(d.get("quant_method", "gptq")),
            sym=bool(d.get("sym", True)),
        )

    @classmethod
    def from_file(cls, path: str) -> "QuantConfig":
        with open(path) as f:
            return cls.from_dict(json.load(f))


def _torch():
    import torch

    return torch


def _identity_groups(g_idx: np.ndarray, gs: int) -> bool:
    return bool(np.array_equal(g_idx, np.arange(g_idx.size, dtype=np.int64) // gs))


def check_gptq_tensors(qweight, scales, group_size: int, qzeros=None, g_idx=None):
    """Validate a GPTQ linear's checkpoint tensors before they reach the
    kernels (which take bare pointers): qweight 32-bit [K/8, N], scales f16
    [K/group_size, N] (the reference reads them as f16 pairs,
    src/shaders/gptq_matvec.wgsl:5-9; other dtypes are refused, not
    converted), qzeros 32-bit [K/group_size, N/8], g_idx [K]. Returns
    (qweight u32, scales u16 bits, qzeros u32 or None, g_idx or None) as
    contiguous arrays."""
    qw = np.ascontiguousarray(qweight)
    if qw.ndim != 2 or qw.dtype.itemsize != 4 or qw.dtype.kind not in "iu":
        raise ValueError(f"qweight: {qw.dtype} {qw.shape}, need a 2-D int32/uint32 [K/8, N]")
    K, N = qw.shape[0] * 8, qw.shape[1]
    if group_size not in (64, 128, 256) or K % group_size:
        raise ValueError(f"group_size {group_size} with K={K} (group sizes 64, 128, 256 dividing K)")
    G = K // group_size
    sc = np.ascontiguousarray(scales)
    if sc.dtype not in (np.float16, np.uint16):
        raise ValueError(f"scales: dtype {sc.dtype}, need float16 (convert the checkpoint's scales explicitly)")
    if sc.shape != (G, N):
        raise ValueError(f"scales: shape {sc.shape}, need {(G, N)}")
    qz = None
    if qzeros is not None:
        qz = np.ascontiguousarray(qzeros)
        if qz.dtype.itemsize != 4 or qz.dtype.kind not in "iu" or qz.shape != (G, N // 8) or N % 8:
            raise ValueError(f"qzeros: {qz.dtype} {qz.shape}, need int32/uint32 {(G, N // 8)}")
        qz = qz.view(np.uint32)
    gi = None
    if g_idx is not None:
        gi = np.ascontiguousarray(g_idx)
        if gi.ndim != 1 or gi.size != K or gi.dtype.kind not in "iu":
            raise ValueError(f"g_idx: {gi.dtype} {gi.shape}, need an integer vector of length K={K}")
    return qw.view(np.uint32), sc.view(np.uint16), qz, gi


@dataclass
class GptqWeight:
    """One GPTQ int4 linear resident in HBM.

    qweight: int32 tensor, [K/8, N] (bit pattern of the u32 words) or, with
             ST_FLAG_TILED in flags, the tiled layout of st_gptq_i4_repack
    scales:  float16 tensor [G, N]
    qzeros:  int32 tensor [G, N/8] or None (symmetric z = 8)
    perm:    int32 tensor [K] or None (act-order: qweight is the sorted copy)
    """

    qweight: object
    scales: object
    qzeros: object
    perm: object
    K: int
    N: int
    group_size: int
    flags: int = 0

    @classmethod
    def upload(cls, gpu, qweight: np.ndarray, scales: np.ndarray, group_size: int = 128,
               qzeros: np.ndarray | None = None, g_idx: np.ndarray | None = None,
               zeros_plus_one: bool = False, tiled: bool = True,
               drop_symmetric_zeros: bool = True) -> "GptqWeight":
        """Upload the checkpoint tensors verbatim (src/weights.rs:398); for an
        act-order g_idx, sort rows by group on the device; with `tiled`,
        repack qweight into the decode kernels' tiled layout (values
        unchanged); otherwise keep the [K/8, N] reference layout.

        Symmetric checkpoints store every zero point as 8 (7 in the AutoGPTQ
        v1 z - 1 convention): with `drop_symmetric_zeros` such qzeros are not
        uploaded, and the kernels use their implicit z = 8, which is the
        reference's own convention (it never reads qzeros,
        src/weights.rs:372-374). The dequantized values are the same bit for
        bit; the decode kernels skip the zero-point table they would
        otherwise build before their first weight load."""
        torch = gpu.torch
        qw, sc, qzeros, g_idx = check_gptq_tensors(qweight, scales, group_size, qzeros, g_idx)
        if drop_symmetric_zeros and qzeros is not None:
            z = np.ascontiguousarray(qzeros).view(np.uint32)
            if np.all(z == (0x77777777 if zeros_plus_one else 0x88888888)):
                qzeros, zeros_plus_one = None, False
        K, N = qw.shape[0] * 8, qw.shape[1]
        d_qw = gpu.upload_array(qw.view(np.int32), torch.int32)
        d_sc = gpu.upload_array(sc.view(np.float16), torch.float16)
        d_qz = None if qzeros is None else gpu.upload_array(qzeros.view(np.int32), torch.int32)
        d_perm = None
        if g_idx is not None and not _identity_groups(np.asarray(g_idx), group_size):
            d_gi = gpu.upload_array(np.ascontiguousarray(g_idx, dtype=np.int32), torch.int32)
            sorted_qw = torch.empty_like(d_qw)
            d_perm = torch.empty(K, dtype=torch.int32, device=gpu.device)
            gpu.sync_stream()
            call("st_gptq_i4_act_order", gpu.handle, d_qw.data_ptr(), d_gi.data_ptr(), sorted_qw.data_ptr(),
                 d_perm.data_ptr(), K, N, group_size)
            d_qw = sorted_qw
        flags = ST_FLAG_ZEROS_PLUS_ONE if zeros_plus_one else 0
        if tiled:
            words = lib().st_gptq_i4_tiled_words(K, N, group_size)
            d_t = torch.empty(words, dtype=torch.int32, device=gpu.device)
            gpu.sync_stream()
            call("st_gptq_i4_repack", gpu.handle, d_qw.data_ptr(), d_t.data_ptr(), K, N, group_size)
            d_qw = d_t
            flags |= ST_FLAG_TILED
        return cls(d_qw, d_sc, d_qz, d_perm, K, N, group_size, flags)

    @classmethod
    def cat(cls, parts: list) -> "GptqWeight":
        """Concatenate linears that share their input along N (q/k/v, or any
        projections of the same x) into one: one launch instead of several,
        outputs side by side in y. Dequantized values are unchanged: in the
        tiled layout each 16-column tile is a contiguous run of words, so the
        tiled buffers simply follow one another; in the [K/8, N] layout the
        columns do. Needs equal K, group size, flags and act-order
        permutation, qzeros on all parts or none, and N % 16 == 0 for all
        parts but the last."""
        torch = _torch()
        p0 = parts[0]
        for p in parts:
            if (p.K, p.group_size, p.flags) != (p0.K, p0.group_size, p0.flags):
                raise ValueError("GptqWeight.cat: parts differ in K, group size or flags")
            if (p.qzeros is None) != (p0.qzeros is None) or (p.perm is None) != (p0.perm is None):
                raise ValueError("GptqWeight.cat: qzeros / act-order present on some parts only")
            if p.perm is not None and not torch.equal(p.perm, p0.perm):
                raise ValueError("GptqWeight.cat: parts have different act-order permutations")
        for p in parts[:-1]:
            if p.N % 16:
                raise ValueError(f"GptqWeight.cat: N={p.N} not a multiple of 16 before the last part")
        if p0.tiled:
            qw = torch.cat([p.qweight.reshape(-1) for p in parts])
        else:
            qw = torch.cat([p.qweight.reshape(p.K // 8, p.N) for p in parts], dim=1).contiguous()
        sc = torch.cat([p.scales.reshape(p.K // p.group_size, p.N) for p in parts], dim=1).contiguous()
        qz = None
        if p0.qzeros is not None:
            qz = torch.cat([p.qzeros.reshape(p.K // p.group_size, p.N // 8) for p in parts], dim=1).contiguous()
        return cls(qw, sc, qz, p0.perm, p0.K, sum(p.N for p in parts), p0.group_size, p0.flags)

    @property
    def tiled(self) -> bool:
        return bool(self.flags & ST_FLAG_TILED)

    @property
    def nbytes(self) -> int:
        n = self.qweight.numel() * 4 + self.scales.numel() * 2
        if self.qzeros is not None:
            n += self.qzeros.numel() * 4
        if self.perm is not None:
            n += self.perm.numel() * 4
        return n


@dataclass
class Int8Weight:
    """INT8 symmetric per-output-channel weight: w int8 [N, K] row-major or,
    with ST_FLAG_TILED in flags, the tiled layout of st_int8_repack; scale
    f32 [N]."""

    w: object
    scale: object
    K: int
    N: int
    flags: int = 0

    @classmethod
    def upload(cls, gpu, w: np.ndarray, scale: np.ndarray, tiled: bool = True) -> "Int8Weight":
        torch = gpu.torch
        w = np.ascontiguousarray(w, dtype=np.int8)
        N, K = w.shape
        d_w = gpu.upload_array(w, torch.int8)
        flags = 0
        if tiled:
            d_t = torch.empty(lib().st_int8_tiled_bytes(K, N), dtype=torch.int8, device=gpu.device)
            gpu.sync_stream()
            call("st_int8_repack", gpu.handle, d_w.data_ptr(), d_t.data_ptr(), K, N)
            d_w, flags = d_t, ST_FLAG_TILED
        return cls(d_w, gpu.upload_array(np.ascontiguousarray(scale, dtype=np.float32), torch.float32), K, N, flags)

    @property
    def nbytes(self) -> int:
        return self.w.numel() + self.scale.numel() * 4
