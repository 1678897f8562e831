"""Static-shape, graph-captured B=1 greedy decode for Mistral/Llama-shaped HF models.

The reference decodes through HF ``generate``: per token, Python walks 32
layers, each patched projection launches one Triton GEMV and the cache
dequantizes its whole cold store (leankv/teal/patching.py:169-177,
leankv/turboquant/cache.py:124-127, scripts/benchmark.py:68-99).  Here one
decode step is a fixed sequence of launches on static buffers, with the token
position kept on the device, captured once into a HIP graph and replayed per
token:

  per layer:  RMSNorm -> TEAL sparse q/k/v GEMV -> RoPE -> cache append
              (quantize the token leaving the fp16 window) -> packed-KV
              attention -> TEAL sparse o_proj -> residual -> RMSNorm ->
              fused TEAL gate/up + SwiGLU -> TEAL sparse down -> residual
  then:       final RMSNorm -> dense lm_head -> argmax (next token on device)

``DenseEngine`` is the same loop with dense fp16 projections (torch F.linear)
and an fp16 KV cache (torch SDPA), the MI355X counterpart of the reference's
dense fp16 baseline (scripts/raw_baseline.py), also graph-captured.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import kernels as _k
from .turboquant.cache import TurboQuantCache


def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """HF MistralRMSNorm: fp32 variance, normalise, cast back, scale (modeling_mistral.py:190-197)."""
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return w * h.to(x.dtype)


def _rot_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class _Base:
    def __init__(self, model, max_len: int):
        cfg = model.config
        self.model = model
        self.cfg = cfg
        self.dev = model.device
        self.L = cfg.num_hidden_layers
        self.H = cfg.num_attention_heads
        self.Hkv = cfg.num_key_value_heads
        self.D = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        self.hidden = cfg.hidden_size
        self.eps = cfg.rms_norm_eps
        self.max_len = max_len
        self.scale = 1.0 / math.sqrt(self.D)
        layers = model.model.layers
        self.layers = layers
        # RoPE tables for every position, computed by the model's own rotary module
        with torch.no_grad():
            pos = torch.arange(max_len, device=self.dev).unsqueeze(0)
            dummy = torch.zeros(1, 1, self.D, device=self.dev, dtype=torch.float16)
            cos, sin = model.model.rotary_emb(dummy, pos)
        self.cos = cos[0].contiguous()  # [max_len, D] fp16
        self.sin = sin[0].contiguous()
        self.tok = torch.zeros(1, dtype=torch.long, device=self.dev)
        self.pos64 = torch.zeros(1, dtype=torch.long, device=self.dev)
        self.logits = torch.zeros(cfg.vocab_size, dtype=torch.float16, device=self.dev)
        self.graph = None

    def _rope(self, q, k):
        cos = self.cos.index_select(0, self.pos64)  # [1, D]
        sin = self.sin.index_select(0, self.pos64)
        q = q * cos + _rot_half(q) * sin
        k = k * cos + _rot_half(k) * sin
        return q, k

    def _finish(self, x):
        x = _rms(x, self.model.model.norm.weight, self.eps)
        self.logits.copy_(F.linear(x, self.model.lm_head.weight).view(-1))
        self.tok.copy_(torch.argmax(self.logits).view(1))
        self.pos64.add_(1)

    def capture(self, warmup: int = 0) -> None:
        """Capture one decode step into a HIP graph (run one eager step first)."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                self._step()
        torch.cuda.current_stream().wait_stream(s)
        self.graph = g

    def step(self) -> None:
        if self.graph is not None:
            self.graph.replay()
        else:
            self._step()

    @torch.no_grad()
    def generate(self, n: int) -> list:
        out = []
        for _ in range(n):
            self.step()
            out.append(self.tok.clone())
        return [int(t) for t in torch.cat(out).tolist()]


class LeanKVEngine(_Base):
    """TEAL sparse projections + TurboQuant packed KV, HIP kernels, one graph per step."""

    def __init__(self, model, cache: TurboQuantCache, max_len: int):
        super().__init__(model, max_len)
        self.cache = cache
        if cache.cold_capacity(0) < max_len - cache.hot_buffer_size:
            raise ValueError("TurboQuantCache cold capacity %d < max_len - hot" % cache.cold_capacity(0))
        self.pos32 = torch.zeros(1, dtype=torch.int32, device=self.dev)
        self.len32 = torch.zeros(1, dtype=torch.int32, device=self.dev)
        self.proj = []
        for layer in self.layers:
            ent = {}
            for name, mod in (("q", layer.self_attn.q_proj), ("k", layer.self_attn.k_proj),
                              ("v", layer.self_attn.v_proj), ("o", layer.self_attn.o_proj),
                              ("gate", layer.mlp.gate_proj), ("up", layer.mlp.up_proj),
                              ("down", layer.mlp.down_proj)):
                t = getattr(mod, "_teal_threshold", None)
                ent[name] = (mod.weight, t)
            self.proj.append(ent)
        # static activations
        d = self.dev
        f16 = torch.float16
        self.q = torch.empty(self.H * self.D, dtype=f16, device=d)
        self.k = torch.empty(self.Hkv * self.D, dtype=f16, device=d)
        self.v = torch.empty(self.Hkv * self.D, dtype=f16, device=d)
        self.attn = torch.empty(1, self.H, self.D, dtype=f16, device=d)
        self.o = torch.empty(self.hidden, dtype=f16, device=d)
        self.m = torch.empty(self.cfg.intermediate_size, dtype=f16, device=d)
        self.dn = torch.empty(self.hidden, dtype=f16, device=d)
        self.x = torch.empty(1, self.hidden, dtype=f16, device=d)
        self.attn_ws = torch.zeros(_k.decode_attn_workspace_bytes(1, self.H, self.Hkv, max_len), dtype=torch.uint8,
                                   device=d)

    def _lin(self, x, w, t, out):
        if t is not None and t > 0:
            return _k.sparse_gemv_out(x, w, t, out)
        out.copy_(F.linear(x.view(1, -1), w).view(-1))
        return out

    def start(self, first_token: torch.Tensor, length: int) -> None:
        """Set the token to feed next and the cache length (after prefill)."""
        self.tok.copy_(first_token.view(1))
        self.pos64.fill_(length)

    def _step(self) -> None:
        c = self.cache
        x = self.model.model.embed_tokens.weight.index_select(0, self.tok)  # [1, hidden]
        self.pos32.copy_(self.pos64)
        self.len32.copy_(self.pos64 + 1)
        for i, layer in enumerate(self.layers):
            p = self.proj[i]
            h = _rms(x, layer.input_layernorm.weight, self.eps)
            self._lin(h, *p["q"], self.q)
            self._lin(h, *p["k"], self.k)
            self._lin(h, *p["v"], self.v)
            q, k = self._rope(self.q.view(1, self.H, self.D), self.k.view(1, self.Hkv, self.D))
            _k.tq_cache_append(k.contiguous(), self.v.view(1, self.Hkv, self.D), c._k_hot[i], c._v_hot[i],
                               c._k_codes[i], c._k_norms[i], c._v_codes[i], c._v_norms[i], c.PiK[i], c.PiV[i],
                               c.decision_boundaries, c.bits, self.pos32)
            _k.tq_decode_attn_out(q.contiguous(), c._k_codes[i], c._k_norms[i], c._v_codes[i], c._v_norms[i],
                                  c._k_hot[i], c._v_hot[i], c.PiK[i], c.PiV[i], c.centroids, c.bits, self.len32,
                                  self.max_len, self.scale, self.attn, self.attn_ws)
            self._lin(self.attn.view(-1), *p["o"], self.o)
            x = x + self.o.view(1, -1)
            h = _rms(x, layer.post_attention_layernorm.weight, self.eps)
            wg, tg = p["gate"]
            wu, tu = p["up"]
            if tg and tu:
                _k.sparse_gateup_swiglu_out(h, wg, wu, tg, tu, self.m)
            else:
                g = F.linear(h, wg) if not tg else _k.sparse_gemv(h, wg, tg).view(1, -1)
                u = F.linear(h, wu) if not tu else _k.sparse_gemv(h, wu, tu).view(1, -1)
                self.m.copy_((F.silu(g) * u).view(-1))
            self._lin(self.m, *p["down"], self.dn)
            x = x + self.dn.view(1, -1)
        self._finish(x)


class DenseEngine(_Base):
    """Dense fp16 projections (torch F.linear) + fp16 KV cache + SDPA, graph-captured."""

    def __init__(self, model, max_len: int):
        super().__init__(model, max_len)
        d = self.dev
        self.K = [torch.zeros(1, self.Hkv, max_len, self.D, dtype=torch.float16, device=d) for _ in range(self.L)]
        self.V = [torch.zeros_like(self.K[0]) for _ in range(self.L)]
        self.ar = torch.arange(max_len, device=d)

    def load_cache(self, past_key_values) -> int:
        """Copy a prefilled HF DynamicCache into the static fp16 buffers; returns its length."""
        n = 0
        for i in range(self.L):
            lay = past_key_values.layers[i]
            k, v = lay.keys, lay.values
            n = k.shape[2]
            self.K[i][:, :, :n] = k
            self.V[i][:, :, :n] = v
        return n

    def start(self, first_token: torch.Tensor, length: int) -> None:
        self.tok.copy_(first_token.view(1))
        self.pos64.fill_(length)

    def _step(self) -> None:
        x = self.model.model.embed_tokens.weight.index_select(0, self.tok)
        mask = (self.ar <= self.pos64).view(1, 1, 1, -1)
        for i, layer in enumerate(self.layers):
            at = layer.self_attn
            h = _rms(x, layer.input_layernorm.weight, self.eps)
            q = F.linear(h, at.q_proj.weight).view(1, self.H, self.D)
            k = F.linear(h, at.k_proj.weight).view(1, self.Hkv, self.D)
            v = F.linear(h, at.v_proj.weight).view(1, self.Hkv, self.D)
            q, k = self._rope(q, k)
            self.K[i].index_copy_(2, self.pos64, k.view(1, self.Hkv, 1, self.D))
            self.V[i].index_copy_(2, self.pos64, v.view(1, self.Hkv, 1, self.D))
            a = F.scaled_dot_product_attention(q.view(1, self.H, 1, self.D), self.K[i], self.V[i], attn_mask=mask,
                                               enable_gqa=True)
            x = x + F.linear(a.reshape(1, -1), at.o_proj.weight)
            h = _rms(x, layer.post_attention_layernorm.weight, self.eps)
            mlp = layer.mlp
            x = x + F.linear(F.silu(F.linear(h, mlp.gate_proj.weight)) * F.linear(h, mlp.up_proj.weight),
                             mlp.down_proj.weight)
        self._finish(x)


# Mistral-7B-v0.3 shape (configs/mistral7b.yaml in the reference).
MISTRAL_7B = dict(vocab_size=32768, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                  num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=32768,
                  rope_theta=1e6, rms_norm_eps=1e-5)


@torch.no_grad()
def random_mistral(device="cuda", seed: int = 0, **overrides):
    """Random-init fp16 MistralForCausalLM (weights ~N(0, 0.02), norms 1) built directly on `device`."""
    from transformers import MistralConfig, MistralForCausalLM

    kw = dict(MISTRAL_7B)
    kw.update(overrides)
    cfg = MistralConfig(**kw)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(seed)
    with torch.device(device):
        model = MistralForCausalLM(cfg).to(torch.float16)
    gen = torch.Generator(device=device).manual_seed(seed)
    for name, p in model.named_parameters():
        if p.dim() == 2:
            p.copy_(torch.randn(p.shape, generator=gen, device=device, dtype=torch.float32).mul_(0.02).to(p.dtype))
        else:
            p.fill_(1.0)
    model.eval()
    return model
