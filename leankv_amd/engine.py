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

import ctypes
import math

import torch
import torch.nn.functional as F

from . import _lib
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
    """TEAL sparse projections + TurboQuant packed KV through the fused C decode step.

    Per token: lkv_decode_begin, lkv_decode_evict (the token leaving every
    layer's hot window, one launch), lkv_decode_layer_step per layer (8
    kernels: q|k|v GEMV with the RMSNorm prologue, attention split with the
    q|k|v sums, RoPE, ring append and query rotation in its prologue, combine,
    o_proj, residual, gate|up GEMV with the RMSNorm prologue, down GEMV with
    the SwiGLU prologue, residual) and
    lkv_decode_head (lm_head GEMV, logits, argmax), captured into one graph.

    Projections patched by apply_teal already hold their weight column-major
    (leankv/teal/patching.py:171); unpatched ones get a column-major copy and
    threshold 0 (dense).  lm_head gets a column-major copy.
    """

    def __init__(self, model, cache: TurboQuantCache, max_len: int):
        super().__init__(model, max_len)
        self.cache = cache
        if cache.cold_capacity(0) < max_len - cache.hot_buffer_size:
            raise ValueError("TurboQuantCache cold capacity %d < max_len - hot" % cache.cold_capacity(0))
        if self.D != 128:
            raise ValueError("the fused decode step needs head_dim 128, got %d" % self.D)
        lib = _lib.load()
        d = self.dev
        self._keep = []  # tensors whose pointers the C structs hold
        self.dims = _lib.DecodeDims(
            hidden=self.hidden, ffn=self.cfg.intermediate_size, vocab=self.cfg.vocab_size, n_heads=self.H,
            n_kv_heads=self.Hkv, max_len=max_len, cap=cache.cold_capacity(0), hot_cap=cache.hot_buffer_size,
            bits=cache.bits, eps=self.eps, scale=self.scale,
            bounds=self._hold(cache.decision_boundaries.to(d, torch.float32).contiguous()),
            centroids=self._hold(cache.centroids.to(d, torch.float32).contiguous()),
            rope_cos=self._hold(self.cos), rope_sin=self._hold(self.sin))
        self.layer_structs = []
        self.thresholds = []
        for i, layer in enumerate(self.layers):
            at, mlp = layer.self_attn, layer.mlp
            w, t = {}, {}
            for name, mod in (("q", at.q_proj), ("k", at.k_proj), ("v", at.v_proj), ("o", at.o_proj),
                              ("g", mlp.gate_proj), ("u", mlp.up_proj), ("d", mlp.down_proj)):
                if getattr(mod, "bias", None) is not None:
                    raise ValueError("the fused decode step has no projection bias")
                th = getattr(mod, "_teal_threshold", None)
                t[name] = float(th) if th else 0.0
                w[name] = self._hold(_colmajor(mod.weight))
            self.thresholds.append(t)
            self.layer_structs.append(_lib.DecodeLayer(
                input_norm=self._hold(layer.input_layernorm.weight.detach()),
                post_norm=self._hold(layer.post_attention_layernorm.weight.detach()),
                wq=w["q"], wk=w["k"], wv=w["v"], wo=w["o"], wg=w["g"], wu=w["u"], wd=w["d"],
                tq=t["q"], tk=t["k"], tv=t["v"], to=t["o"], tg=t["g"], tu=t["u"], td=t["d"],
                k_codes=self._hold(cache._k_codes[i]), k_norms=self._hold(cache._k_norms[i]),
                v_codes=self._hold(cache._v_codes[i]), v_norms=self._hold(cache._v_norms[i]),
                k_hot=self._hold(cache._k_hot[i]), v_hot=self._hold(cache._v_hot[i]),
                PiK=self._hold(cache.PiK[i].contiguous()), PiV=self._hold(cache.PiV[i].contiguous())))
        self.layer_table = (_lib.DecodeLayer * len(self.layer_structs))(*self.layer_structs)
        self.final_norm = model.model.norm.weight.detach()
        self.lm_head_cm = model.lm_head.weight.detach().t().contiguous()  # [hidden][vocab]
        nbytes = lib.lkv_decode_workspace_bytes(ctypes.byref(self.dims))
        if nbytes == 0:
            raise _lib.LeanKVError("lkv_decode_workspace_bytes rejected the model shape: %s" % _lib.last_error())
        self.ws = torch.empty(nbytes, dtype=torch.uint8, device=d)
        self.x = torch.empty(self.hidden, dtype=torch.float16, device=d)

    def _hold(self, t: torch.Tensor) -> int:
        if not t.is_cuda:
            raise _lib.LeanKVError("decode state must live on the GPU")
        self._keep.append(t)
        return t.data_ptr()

    def start(self, first_token: torch.Tensor, length: int) -> None:
        """Set the token to feed next and its position (the cache length after prefill)."""
        self.tok.copy_(first_token.view(1))
        self.pos64.fill_(length)

    def _step(self) -> None:
        lib = _lib.load()
        st = _lib.stream_handle(self.dev)
        ws, nb = self.ws.data_ptr(), self.ws.numel()
        dims = ctypes.byref(self.dims)
        _lib.check(lib.lkv_decode_begin(dims, self.model.model.embed_tokens.weight.data_ptr(), self.tok.data_ptr(),
                                        self.pos64.data_ptr(), self.x.data_ptr(), ws, nb, st), "lkv_decode_begin")
        _lib.check(lib.lkv_decode_evict(dims, self.layer_table, len(self.layer_structs), ws, nb, st),
                   "lkv_decode_evict")
        for ls in self.layer_structs:
            _lib.check(lib.lkv_decode_layer_step(dims, ctypes.byref(ls), self.x.data_ptr(), ws, nb, st),
                       "lkv_decode_layer_step")
        _lib.check(lib.lkv_decode_head(dims, self.final_norm.data_ptr(), self.lm_head_cm.data_ptr(),
                                       self.x.data_ptr(), self.logits.data_ptr(), self.tok.data_ptr(),
                                       self.pos64.data_ptr(), ws, nb, st), "lkv_decode_head")


def _colmajor(w: torch.Tensor) -> torch.Tensor:
    """[Z][N] row-major view of a weight W[N, Z] (column-major storage), copying only if needed."""
    w = w.detach()
    wt = w.t()
    return wt if wt.is_contiguous() else wt.contiguous()


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
