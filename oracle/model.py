"""CPU reference decode of a Mistral-shaped model with TEAL + TurboQuant (test infrastructure).

Restates, in torch-CPU fp32 with fp16 rounding at the points where the
reference's fp16 GPU run stores tensors:
  transformers/models/mistral/modeling_mistral.py  RMSNorm (:180-197), rotary
      embedding + apply_rotary_pos_emb, GQA attention (:139-178), MLP (:46-47),
      decoder layer residual order
  leankv/teal/patching.py:101-125, 169-177   per-projection thresholds; the
      Triton path compares |x| (fp16) with the fp32 threshold (sparse_gemv.py:82)
  leankv/turboquant/cache.py:84-189           hot window of 64 fp16 tokens,
      older tokens quantized as fp32, attention over dequant(cold).fp16 ++ hot
Every projection output is rounded to fp16 (the kernel writes fp16).
"""

from __future__ import annotations

import math
import time

import torch

from . import turboquant as oq

PROJS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def f16(t: torch.Tensor) -> torch.Tensor:
    """Round to fp16 and return as fp32 (a value the fp16 GPU run would store)."""
    return t.to(torch.float16).to(torch.float32)


class RefModel:
    def __init__(self, state: dict, cfg, thresholds: dict | None, bits: int = 3, hot: int = 64, seed: int = 42,
                 acc_dtype: torch.dtype = torch.float64):
        """acc_dtype: accumulation dtype of the projections (fp64 = truth; fp32 = timing baseline)."""
        self.acc = acc_dtype
        self._acc_w = {}
        self.cfg = cfg
        self.sd = {k: v.detach().to("cpu", torch.float32) for k, v in state.items()}
        self.th = thresholds or {}
        self.L = cfg.num_hidden_layers
        self.H = cfg.num_attention_heads
        self.Hkv = cfg.num_key_value_heads
        self.D = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        self.eps = cfg.rms_norm_eps
        self.theta = getattr(cfg, "rope_theta", None) or cfg.rope_parameters["rope_theta"]
        c, b = oq.codebook_tensors(bits)
        self.t_layers = 0.0  # seconds spent in the decoder layers / in embedding + final norm + lm_head
        self.t_head = 0.0
        self.caches = [oq.CacheRef(oq.rotation_matrix(self.D, seed + 2 * i), oq.rotation_matrix(self.D, seed + 2 * i + 1),
                                   c, b, bits, hot) for i in range(self.L)]
        self.pos = 0

    # ---------------------------------------------------------------- pieces
    def _w(self, name):
        return self.sd[name]

    def _wacc(self, name):
        """Weight in the accumulation dtype, converted once (a full-width fp64 step would otherwise
        re-convert ~1 GB of weights)."""
        w = self._acc_w.get(name)
        if w is None:
            w = self._acc_w[name] = self._w(name).to(self.acc).T.contiguous()
        return w

    def _lin(self, x, layer, proj, mod):
        """x fp32 (fp16 values) [S, Z] -> fp16-rounded y [S, N]; TEAL mask only at single-token decode."""
        Wt = self._wacc("model.layers.%d.%s.%s.weight" % (layer, mod, proj))
        t = self.th.get(layer, {}).get(proj, 0.0)
        if t > 0 and x.shape[0] == 1:
            x = torch.where(x.abs() > torch.tensor(t, dtype=torch.float32), x, torch.zeros_like(x))
        return f16(x.to(self.acc).matmul(Wt).float())

    def _rms(self, x, w):
        var = x.pow(2).mean(-1, keepdim=True)
        return f16(w * f16(x * torch.rsqrt(var + self.eps)))

    def _rope(self, pos):
        inv = 1.0 / (self.theta ** (torch.arange(0, self.D, 2, dtype=torch.int64).float() / self.D))
        fr = torch.outer(pos.float(), inv)
        emb = torch.cat([fr, fr], dim=-1)
        return f16(emb.cos()), f16(emb.sin())

    @staticmethod
    def _rot_half(x):
        h = x.shape[-1] // 2
        return torch.cat([-x[..., h:], x[..., :h]], dim=-1)

    # ---------------------------------------------------------------- forward
    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        """Run S new tokens (prefill if S > 1); returns fp32 logits of the last token."""
        t0 = time.perf_counter()
        S = ids.shape[0]
        pos = torch.arange(self.pos, self.pos + S)
        cos, sin = self._rope(pos)
        x = f16(self._w("model.embed_tokens.weight")[ids])
        t1 = time.perf_counter()
        for i in range(self.L):
            p = "model.layers.%d." % i
            h = self._rms(x, self._w(p + "input_layernorm.weight"))
            q = self._lin(h, i, "q_proj", "self_attn").view(S, self.H, self.D).transpose(0, 1)
            k = self._lin(h, i, "k_proj", "self_attn").view(S, self.Hkv, self.D).transpose(0, 1)
            v = self._lin(h, i, "v_proj", "self_attn").view(S, self.Hkv, self.D).transpose(0, 1)
            q = f16(f16(q * cos) + f16(self._rot_half(q) * sin))
            k = f16(f16(k * cos) + f16(self._rot_half(k) * sin))
            K, V = self.caches[i].update(k.unsqueeze(0).half(), v.unsqueeze(0).half())
            K, V = K[0].float(), V[0].float()
            G = self.H // self.Hkv
            Kx, Vx = K.repeat_interleave(G, 0), V.repeat_interleave(G, 0)
            s = q.double().matmul(Kx.double().transpose(-1, -2)) / math.sqrt(self.D)
            T = K.shape[1]
            causal = torch.arange(T)[None, :] <= (T - S + torch.arange(S))[:, None]
            s = s.masked_fill(~causal, float("-inf"))
            a = f16(torch.softmax(s, -1).matmul(Vx.double()).float())
            a = a.transpose(0, 1).reshape(S, self.H * self.D)
            x = f16(x + self._lin(a, i, "o_proj", "self_attn"))
            h = self._rms(x, self._w(p + "post_attention_layernorm.weight"))
            g = self._lin(h, i, "gate_proj", "mlp")
            u = self._lin(h, i, "up_proj", "mlp")
            m = f16(f16(g / (1 + torch.exp(-g))) * u)
            x = f16(x + self._lin(m, i, "down_proj", "mlp"))
        t2 = time.perf_counter()
        x = self._rms(x, self._w("model.norm.weight"))
        self.pos += S
        out = x[-1:].to(self.acc).matmul(self._wacc("lm_head.weight")).float()[0]
        t3 = time.perf_counter()
        self.t_layers += t2 - t1
        self.t_head += (t1 - t0) + (t3 - t2)
        return out
