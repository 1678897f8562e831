"""CPU restatement of TurboQuant MSE + its KV cache + decode attention (test infrastructure).

References (under /root/reference, read as text):
  leankv/turboquant/rotation.py:12-29   generate_rotation_matrix (randn + QR + sign fix)
  leankv/turboquant/rotation.py:45-52   rotate_forward x@Pi^T, rotate_backward y@Pi
  leankv/turboquant/quantizer.py:38-62  _pack_indices
  leankv/turboquant/quantizer.py:65-85  _unpack_indices
  leankv/turboquant/quantizer.py:119-129 TurboQuantMSE.quantize
  leankv/turboquant/quantizer.py:131-137 TurboQuantMSE.dequantize
  leankv/turboquant/rotation.py:32-42   generate_qjl_matrix (seeded i.i.d. N(0,1))
  leankv/turboquant/quantizer.py:144-237 TurboQuantProd (sign packing, quantize, dequantize)
  leankv/turboquant/cache.py:84-189     TurboQuantCache.update / flush / full cache
  transformers/integrations/sdpa_attention.py:79-105  GQA SDPA on the returned K/V
  transformers/masking_utils.py causal_mask_function   causal mask with the cache offset (prefill)
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tests", "golden")


def load_codebook(bits: int, d: int = 128) -> dict:
    """Golden codebook written by the reference's own solver (make_golden.py)."""
    with open(os.path.join(GOLDEN, "codebook_d%d_b%d.json" % (d, bits))) as f:
        return json.load(f)


def codebook_tensors(bits: int):
    """(centroids fp32, boundaries fp32) as get_codebook_tensors does (codebook.py:163-170)."""
    cb = load_codebook(bits)
    return (torch.tensor(cb["centroids"], dtype=torch.float32),
            torch.tensor(cb["boundaries"], dtype=torch.float32))


def rotation_matrix(d: int, seed: int) -> torch.Tensor:
    """generate_rotation_matrix (rotation.py:12-29) on the CPU, fp32."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    G = torch.randn(d, d, generator=g, dtype=torch.float32)
    Q, R = torch.linalg.qr(G)
    return Q * torch.sign(torch.diag(R)).unsqueeze(0)


def _vals_per_byte(bits: int) -> tuple[int, int]:
    if bits == 1:
        return 8, 1
    if bits == 2:
        return 4, 2
    if bits <= 4:
        return 2, 4
    raise ValueError("bits > 4 are stored unpacked")


def pack_indices(idx: np.ndarray, bits: int) -> np.ndarray:
    """_pack_indices (quantizer.py:38-62): little-end-first fields, 3 bits padded to 4."""
    vpb, pb = _vals_per_byte(bits)
    idx = np.asarray(idx, dtype=np.uint8)
    d = idx.shape[-1]
    pad = (-d) % vpb
    if pad:
        idx = np.concatenate([idx, np.zeros(idx.shape[:-1] + (pad,), np.uint8)], axis=-1)
    r = idx.reshape(idx.shape[:-1] + (-1, vpb)).astype(np.uint32)
    shifts = (np.arange(vpb, dtype=np.uint32) * pb)
    return (r << shifts).sum(axis=-1).astype(np.uint8)


def unpack_indices(packed: np.ndarray, bits: int, d: int) -> np.ndarray:
    """_unpack_indices (quantizer.py:65-85)."""
    vpb, pb = _vals_per_byte(bits)
    p = np.asarray(packed, dtype=np.uint8)[..., None].astype(np.uint32)
    shifts = (np.arange(vpb, dtype=np.uint32) * pb)
    u = (p >> shifts) & ((1 << pb) - 1)
    return u.reshape(p.shape[:-2] + (-1,))[..., :d].astype(np.int64)


def quantize(x: torch.Tensor, Pi: torch.Tensor, boundaries: torch.Tensor, bits: int):
    """TurboQuantMSE.quantize (quantizer.py:119-129) with torch CPU ops.

    Returns (packed uint8 ndarray, norms tensor in x's dtype, y fp32 tensor).
    """
    x = x.cpu()
    norms = x.norm(dim=-1)
    x_unit = x / (norms.unsqueeze(-1) + 1e-10)
    y = torch.matmul(x_unit.float(), Pi.T)
    idx = torch.searchsorted(boundaries[1:-1].contiguous(), y.contiguous())
    return pack_indices(idx.numpy(), bits), norms, y


def dequantize(packed: np.ndarray, norms: torch.Tensor, Pi: torch.Tensor, centroids: torch.Tensor,
               bits: int, d: int = 128) -> torch.Tensor:
    """TurboQuantMSE.dequantize (quantizer.py:131-137), fp32."""
    idx = torch.from_numpy(unpack_indices(packed, bits, d))
    y_hat = centroids[idx]
    return torch.matmul(y_hat, Pi) * norms.float().unsqueeze(-1)


def qjl_matrix(d: int, seed: int) -> torch.Tensor:
    """generate_qjl_matrix (rotation.py:32-42): i.i.d. N(0,1) from a seeded CPU generator, fp32."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return torch.randn(d, d, generator=g, dtype=torch.float32)


def pack_signs(proj: np.ndarray) -> np.ndarray:
    """TurboQuantProd._pack_qjl_signs (quantizer.py:181-194): bit i of byte j = [proj[8j + i] > 0]."""
    bits = (np.asarray(proj) > 0).astype(np.uint8)
    d = bits.shape[-1]
    if d % 8:
        bits = np.concatenate([bits, np.zeros(bits.shape[:-1] + (8 - d % 8,), np.uint8)], axis=-1)
    r = bits.reshape(bits.shape[:-1] + (-1, 8)).astype(np.uint32)
    return (r << np.arange(8, dtype=np.uint32)).sum(axis=-1).astype(np.uint8)


def unpack_signs(packed: np.ndarray, d: int = 128) -> np.ndarray:
    """TurboQuantProd._unpack_qjl_signs (quantizer.py:196-204): +1 / -1 float32 per coordinate."""
    p = np.asarray(packed, dtype=np.uint8)[..., None]
    b = (p >> np.arange(8, dtype=np.uint8)) & 1
    return (2.0 * b.reshape(p.shape[:-2] + (-1,))[..., :d] - 1.0).astype(np.float32)


def prod_quantize(x: torch.Tensor, Pi: torch.Tensor, boundaries: torch.Tensor, centroids: torch.Tensor,
                  S: torch.Tensor, mse_bits: int):
    """TurboQuantProd.quantize (quantizer.py:206-222) with torch CPU ops.

    MSE codes and norms at mse_bits, x_hat their dequantization, residual
    r = x - x_hat in fp32, its norm, and the signs of r @ S^T.  Returns
    (packed codes, norms, packed signs, residual norms fp32, r @ S^T fp32).
    """
    x = x.cpu()
    packed, norms, _ = quantize(x, Pi, boundaries, mse_bits)
    x_hat = dequantize(packed, norms, Pi, centroids, mse_bits)
    residual = x - x_hat
    proj = torch.matmul(residual.float(), S.T)
    return packed, norms, pack_signs(proj.numpy()), residual.norm(dim=-1), proj


def prod_dequantize(packed: np.ndarray, norms: torch.Tensor, signs: np.ndarray, rnorms: torch.Tensor,
                    Pi: torch.Tensor, centroids: torch.Tensor, S: torch.Tensor, mse_bits: int,
                    d: int = 128) -> torch.Tensor:
    """TurboQuantProd.dequantize (quantizer.py:224-237), fp32:
    x_mse + (signs @ S) * (sqrt(pi / 2) / d * ||r||)."""
    x_mse = dequantize(packed, norms, Pi, centroids, mse_bits, d)
    x_qjl = torch.matmul(torch.from_numpy(unpack_signs(signs, d)), S)
    x_qjl = x_qjl * ((math.sqrt(math.pi / 2.0) / d) * rnorms.float().unsqueeze(-1))
    return x_mse + x_qjl


class CacheRef:
    """TurboQuantCache (cache.py:35-189) for one layer, CPU, reference semantics.

    update() returns the full K/V the reference hands to attention:
    cat(dequantize(cold).to(fp16), hot) along the sequence axis.
    """

    def __init__(self, PiK, PiV, centroids, boundaries, bits=3, hot=64):
        self.PiK, self.PiV = PiK, PiV
        self.c, self.b = centroids, boundaries
        self.bits, self.hot_size = bits, hot
        self.hot_k = self.hot_v = None
        self.cold_k = []  # list of (packed, norms)
        self.cold_v = []

    def update(self, k: torch.Tensor, v: torch.Tensor):
        k, v = k.to(torch.float16), v.to(torch.float16)
        self.hot_k = k if self.hot_k is None else torch.cat([self.hot_k, k], dim=2)
        self.hot_v = v if self.hot_v is None else torch.cat([self.hot_v, v], dim=2)
        n = self.hot_k.shape[2]
        if n > self.hot_size:
            f = n - self.hot_size
            pk, nk, _ = quantize(self.hot_k[:, :, :f].float(), self.PiK, self.b, self.bits)
            pv, nv, _ = quantize(self.hot_v[:, :, :f].float(), self.PiV, self.b, self.bits)
            self.cold_k.append((pk, nk))
            self.cold_v.append((pv, nv))
            self.hot_k = self.hot_k[:, :, f:].contiguous()
            self.hot_v = self.hot_v[:, :, f:].contiguous()
        return self.full()

    def cold_arrays(self):
        if not self.cold_k:
            return None
        pk = np.concatenate([p for p, _ in self.cold_k], axis=2)
        nk = torch.cat([n for _, n in self.cold_k], dim=2)
        pv = np.concatenate([p for p, _ in self.cold_v], axis=2)
        nv = torch.cat([n for _, n in self.cold_v], dim=2)
        return pk, nk, pv, nv

    def full(self):
        ca = self.cold_arrays()
        if ca is None:
            return self.hot_k, self.hot_v
        pk, nk, pv, nv = ca
        ck = dequantize(pk, nk, self.PiK, self.c, self.bits).to(torch.float16)
        cv = dequantize(pv, nv, self.PiV, self.c, self.bits).to(torch.float16)
        return torch.cat([ck, self.hot_k], dim=2), torch.cat([cv, self.hot_v], dim=2)


def decode_attention(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, scale: float | None = None):
    """Single-query GQA attention in fp64 (sdpa_attention.py:79-105 semantics).

    q [B, Hq, 1, D], K/V [B, Hkv, L, D] -> [B, Hq, 1, D] fp64.  Query head h
    reads kv head h // (Hq / Hkv) (repeat_kv).
    """
    B, Hq, _, D = q.shape
    Hkv = K.shape[1]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    qd = q.double()
    Kd = K.double().repeat_interleave(G, dim=1)
    Vd = V.double().repeat_interleave(G, dim=1)
    s = torch.matmul(qd, Kd.transpose(-1, -2)) * scale
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, Vd)


def prefill_attention(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, scale: float | None = None):
    """Causal GQA attention of the newest S tokens' queries in fp64.

    q [B, Hq, S, D], K/V [B, Hkv, L, D] with L >= S -> [B, Hq, S, D] fp64.  Query i
    sits at position L - S + i and sees keys 0 .. L - S + i: HF's causal mask
    with the cache offset (masking_utils causal_mask_function, kv_idx <= q_idx)
    applied by SDPA (sdpa_attention.py:79-105) to the K/V the cache returns.
    """
    B, Hq, S, D = q.shape
    Hkv, L = K.shape[1], K.shape[2]
    G = Hq // Hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    Kd = K.double().repeat_interleave(G, dim=1)
    Vd = V.double().repeat_interleave(G, dim=1)
    s = torch.matmul(q.double(), Kd.transpose(-1, -2)) * scale
    qpos = torch.arange(S).view(S, 1) + (L - S)
    visible = torch.arange(L).view(1, L) <= qpos
    s = s.masked_fill(~visible, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), Vd)
