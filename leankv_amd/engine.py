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

Two dense fp16 baselines run the same model with an fp16 KV cache, both
graph-captured: ``OwnDenseEngine`` is LeanKVEngine's step on this library's
kernels with every TEAL threshold 0 and the fp16 cache in pages (the strong
baseline), ``DenseEngine`` is torch F.linear + SDPA (the reference's dense
fp16 run, scripts/raw_baseline.py, as torch executes it).
"""

from __future__ import annotations

import ctypes
import math

import torch
import torch.nn.functional as F

from . import _lib
from .turboquant.cache import TurboQuantCache

STEP_BITS = (1, 2, 3, 4)  # code widths the fused B = 1 decode step (lkv_decode_*) is built for


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
        # hist[p]: the token the step at position p produced (written on the device inside the step)
        self.hist = torch.zeros(max_len, dtype=torch.long, device=self.dev)
        self.graph = None
        self._host_pos = None  # position of the next step, tracked on the host to bound it by max_len

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
        self.hist.index_copy_(0, self.pos64, self.tok)
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

    def _set_start(self, first_token: torch.Tensor, length: int) -> None:
        if not 0 <= int(length) < self.max_len:
            raise _lib.LeanKVError("decode start position %d outside the engine's max_len %d"
                                   % (int(length), self.max_len))
        self.tok.copy_(first_token.view(1))
        self.pos64.fill_(int(length))
        self._host_pos = int(length)

    def step(self) -> None:
        """One greedy decode step; the position it writes must stay below max_len (the RoPE table and the
        cache are sized for it), so a step past it raises instead of overwriting the last slot."""
        if self._host_pos is None:
            raise _lib.LeanKVError("call start(first_token, length) before stepping the engine")
        if self._host_pos >= self.max_len:
            raise _lib.LeanKVError("decode position %d reached the engine's max_len %d"
                                   % (self._host_pos, self.max_len))
        if self.graph is not None:
            self.graph.replay()
        else:
            self._step()
        self._host_pos += 1

    @torch.no_grad()
    def generate(self, n: int) -> list:
        if self._host_pos is not None and self._host_pos + n > self.max_len:
            raise _lib.LeanKVError("%d more tokens from position %d exceed the engine's max_len %d"
                                   % (n, self._host_pos, self.max_len))
        p0 = self._host_pos
        for _ in range(n):
            self.step()
        return [int(t) for t in self.hist[p0:p0 + n].tolist()]


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
        self._set_start(first_token, length)

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
                                       self.pos64.data_ptr(), self.hist.data_ptr(), self.hist.numel(), ws, nb, st),
                   "lkv_decode_head")


_HF_RMSNORMS = ("MistralRMSNorm", "LlamaRMSNorm")


class BatchedEngine:
    """One decode step of B > 1 sequences of equal length on a fused TurboQuantCache, captured once and
    replayed as a HIP graph.

    At B > 1 the reference's patched projections run dense F.linear (leankv/teal/patching.py:169-180);
    HF's decoder layer then calls TurboQuantCache.update and the attention function per layer
    (modeling_mistral.py:135-174, cache.py:84-127).  This step makes the same calls in the same order on
    the same modules -- embedding, the (patched) projections, the cache's append and decode-attention
    kernels, o_proj, residual adds, the (patched) MLP and lm_head -- with the position on the device, so the
    whole step replays without the host.  RMSNorm runs as one lkv_rmsnorm launch (the B = 1 step's
    arithmetic) and RoPE as one lkv_rope_f16 launch (HF's fp16 arithmetic bit for bit) instead of HF's
    chains of elementwise kernels (in the reduce of the patched q/k/v launch when there is one, which then
    also writes the new token into the hot ring, the token leaving every layer's window being evicted by one
    launch at the step's start: TurboQuantCache.update's two halves), and each residual add runs with the
    RMSNorm after it in one launch behind the patched o_proj / down_proj product (the same bits as the add and
    lkv_rmsnorm): with the model's RMSNorm modules on lkv_rmsnorm the logits equal the
    HF forward's bit for bit; with HF's torch RMSNorm they differ from it in the last bits of the norms,
    as the B = 1 step's do.  tok [B] is fed, logits [B, vocab] come out; the cache's host counters are the
    caller's to advance (GenerateFastPath does)."""

    def __init__(self, model, cache: TurboQuantCache, B: int):
        import sys

        from . import kernels

        cfg = model.config
        self.model, self.cache, self.B = model, cache, B
        self.dev = model.device
        self.D = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        self.Hq, self.Hkv = cfg.num_attention_heads, cfg.num_key_value_heads
        self.max_len = cache.attn_max_len(0)
        layers = model.model.layers
        attn_module = type(layers[0].self_attn).__module__
        self._rope = sys.modules[attn_module].apply_rotary_pos_emb
        # the standard rotate-half form (modeling_mistral.py:51-81, the same in modeling_llama) runs as one
        # lkv_rope_f16 launch; other model families keep their own function
        self._fused_rope = attn_module.rsplit(".", 1)[-1] in ("modeling_mistral", "modeling_llama") and self.D == 128
        with torch.no_grad():
            pos = torch.arange(self.max_len, device=self.dev).unsqueeze(0)
            dummy = torch.zeros(1, 1, self.D, device=self.dev, dtype=torch.float16)
            cos, sin = model.model.rotary_emb(dummy, pos)
        self.cos, self.sin = cos[0].contiguous(), sin[0].contiguous()  # [max_len, D], the HF forward's values
        self._fused_rope = self._fused_rope and self.cos.dtype == torch.float16 and self.sin.dtype == torch.float16
        # Every layer's q/k/v one launch with RoPE: then that launch writes the new token into the hot ring and
        # one launch per step evicts the tokens leaving every layer's window (tq_cache_append's two halves)
        from .teal.patching import _qkv_fusable

        fus = [_qkv_fusable(l.self_attn, B, torch.float16) for l in layers] if self._fused_rope else [None]
        self._ring = all(f is not None and f[0].shape[0] % 128 == 0 and f[1].shape[0] == self.Hkv * self.D
                         and f[2].shape[0] == self.Hkv * self.D for f in fus)
        self.tok = torch.zeros(B, dtype=torch.long, device=self.dev)
        self.pos64 = torch.zeros(1, dtype=torch.long, device=self.dev)
        self.pos32 = torch.zeros(1, dtype=torch.int32, device=self.dev)  # position of the token fed
        self.len32 = torch.ones(1, dtype=torch.int32, device=self.dev)   # cache length after its append
        self.logits = None
        self.attn = torch.empty(B, self.Hq, self.D, dtype=torch.float16, device=self.dev)
        self.attn_ws = torch.empty(kernels.decode_attn_workspace_bytes(B, self.Hq, self.Hkv, self.max_len),
                                   dtype=torch.uint8, device=self.dev)
        self.graph = None
        self._host_pos = None

    def _layer(self, i: int, layer, x: torch.Tensor, h: torch.Tensor, cos, sin, next_norm):
        """One decoder layer on x (h = its input_layernorm(x)); returns the layer's output and next_norm of it
        (the next layer's input_layernorm, or the model's final norm)."""
        from . import kernels
        from .teal.patching import _qkv_fusable, _qkv_rows

        c, B, D = self.cache, self.B, self.D
        at = layer.self_attn
        residual = x
        # a fused TEAL q/k/v patch: the three products and RoPE on q and k as one launch (with the ring write)
        appended = False
        if self._ring and h.dtype == torch.float16:  # (the step's start evicted every layer's leaving token)
            ws = _qkv_fusable(at, B, h.dtype)
            qp, kp, vp = (torch.empty(B, w.shape[0], dtype=torch.float16, device=self.dev) for w in ws)
            kernels.sparse_gemm_batched_qkv_rope_out(h.reshape(B, -1).contiguous(), list(ws), cos.view(-1),
                                                     sin.view(-1), [qp, kp, vp], c._k_hot[i], c._v_hot[i],
                                                     self.pos32)
            fused = appended = True
        elif (qkv := _qkv_rows(at, h, cos.view(-1), sin.view(-1)) if self._fused_rope else None) is not None:
            qp, kp, vp = qkv
            fused = True
        else:
            qp, kp, vp = at.q_proj(h), at.k_proj(h), at.v_proj(h)
            fused = (self._fused_rope and qp.dtype == torch.float16 and kp.dtype == torch.float16
                     and qp.is_contiguous() and kp.is_contiguous())
            if fused:  # in place on the fresh projection outputs, one launch for both
                kernels.rope_f16_(qp.view(B, self.Hq, D), kp.view(B, self.Hkv, D), cos.view(-1), sin.view(-1))
        q = qp.view(B, 1, -1, D).transpose(1, 2)
        k = kp.view(B, 1, -1, D).transpose(1, 2)
        v = vp.view(B, 1, -1, D).transpose(1, 2)
        if not fused:
            q, k = self._rope(q, k, cos, sin)
        if not appended:
            k16, v16 = k.to(torch.float16), v.to(torch.float16)
            kernels.tq_cache_append(k16.reshape(B, self.Hkv, D).contiguous(),
                                    v16.reshape(B, self.Hkv, D).contiguous(), c._k_hot[i], c._v_hot[i],
                                    c._k_codes[i], c._k_norms[i], c._v_codes[i], c._v_norms[i], c.PiK[i], c.PiV[i],
                                    c.decision_boundaries, c.bits, self.pos32)
        qf = q.reshape(B, self.Hq, D).to(torch.float16).contiguous()
        kernels.tq_decode_attn_out(qf, c._k_codes[i], c._k_norms[i], c._v_codes[i], c._v_norms[i], c._k_hot[i],
                                   c._v_hot[i], c.PiK[i], c.PiV[i], c.centroids, c.bits, self.len32, self.max_len,
                                   float(at.scaling), self.attn, self.attn_ws)
        o = self.attn.view(B, self.Hq, 1, D).transpose(1, 2).contiguous().to(q.dtype).reshape(B, 1, -1)
        x, h = self._residual_proj(at.o_proj, o, residual, layer.post_attention_layernorm)
        return self._residual_mlp(layer.mlp, h, x, next_norm)

    def _residual_proj(self, proj, inp: torch.Tensor, residual: torch.Tensor, norm=None):
        """(x, norm(x)) for x = residual + proj(inp).  A TEAL-patched projection that sends these B rows to the
        batched kernel (threshold 0) runs as one launch with HF's fp16 residual add in its reduce, or, when norm
        is an RMSNorm _norm runs on lkv_rmsnorm, with the add and the norm in one launch after the product: the
        same bits as the projection's forward, torch's add and _norm."""
        from . import kernels
        from .teal.patching import _skinny_dense

        B, w = self.B, getattr(proj, "weight", None)
        if (getattr(proj, "_teal_patched", False) and proj.bias is None and w is not None and w.dim() == 2
                and w.dtype == torch.float16 and inp.dtype == torch.float16 and residual.dtype == torch.float16
                and inp.numel() == B * w.shape[1] and residual.numel() == B * w.shape[0]
                and residual.is_contiguous() and _skinny_dense(B, w.shape[0], w.shape[1])):
            out = torch.empty_like(residual)
            x2 = inp.reshape(B, -1).contiguous()
            if self._lkv_norm(norm, residual) and w.shape[0] <= 8192:
                y = torch.empty_like(residual)
                kernels.sparse_gemm_batched_residual_rmsnorm_out(x2, w, 0.0, residual.view(B, -1), norm.weight,
                                                                 norm.variance_epsilon, out.view(B, -1),
                                                                 y.view(B, -1))
                return out, y
            kernels.sparse_gemm_batched_multi_out(x2, [w], [0.0], [out.view(B, -1)], kernels.EPI_RESIDUAL,
                                                  residual.view(B, -1))
        else:
            out = residual + proj(inp)
        return out, (self._norm(norm, out) if norm is not None else None)

    def _residual_mlp(self, mlp, h: torch.Tensor, residual: torch.Tensor, norm=None):
        """(x, norm(x)) for x = residual + mlp(h).  For a fused TEAL MLP whose gate/up + SwiGLU takes these rows
        as one batched launch, the down projection then runs through _residual_proj: the MLP forward's own
        calls, with the add (and the norm) fused."""
        from .teal.patching import _gateup_rows

        down = getattr(mlp, "down_proj", None)
        if getattr(mlp, "_teal_fused", False) and down is not None:
            a = _gateup_rows(mlp, h)
            if a is not None:
                return self._residual_proj(down, a, residual, norm)
        out = residual + mlp(h)
        return out, (self._norm(norm, out) if norm is not None else None)

    @staticmethod
    def _lkv_norm(mod, x: torch.Tensor) -> bool:
        """Whether _norm runs mod on x as lkv_rmsnorm."""
        w = getattr(mod, "weight", None)
        return (type(mod).__name__ in _HF_RMSNORMS and x.dtype == torch.float16 and w is not None
                and w.dtype == torch.float16 and w.numel() == x.shape[-1] and x.shape[-1] % 8 == 0
                and w.is_contiguous())

    @staticmethod
    def _norm(mod, x: torch.Tensor) -> torch.Tensor:
        """HF's Mistral / Llama RMSNorm on fp16 as one lkv_rmsnorm launch (the summation order of the B = 1
        step's fused RMSNorm; HF's torch RMSNorm runs seven kernels and sums in another order, so its last bits
        can differ), any other norm module as it is."""
        from . import kernels

        if BatchedEngine._lkv_norm(mod, x):
            return kernels.rms_norm(x, mod.weight, mod.variance_epsilon)
        return mod(x)

    def _step(self) -> None:
        from . import kernels

        m = self.model
        x = m.model.embed_tokens(self.tok.view(self.B, 1))
        cos = self.cos.index_select(0, self.pos64).unsqueeze(0)  # [1, 1, D]
        sin = self.sin.index_select(0, self.pos64).unsqueeze(0)
        layers = m.model.layers
        if self._ring:  # the token leaving every layer's hot window, before any layer writes its new one
            c = self.cache
            kernels.tq_cache_evict([(c._k_codes[i], c._k_norms[i], c._v_codes[i], c._v_norms[i], c._k_hot[i],
                                     c._v_hot[i], c.PiK[i], c.PiV[i]) for i in range(len(layers))],
                                   c.decision_boundaries, c.bits, self.pos32)
        h = self._norm(layers[0].input_layernorm, x)
        for i, layer in enumerate(layers):
            nxt = layers[i + 1].input_layernorm if i + 1 < len(layers) else m.model.norm
            x, h = self._layer(i, layer, x, h, cos, sin, nxt)
        logits = m.lm_head(h)
        if self.logits is None:
            self.logits = torch.empty_like(logits)
        self.logits.copy_(logits)
        self.pos64.add_(1)
        self.pos32.add_(1)
        self.len32.add_(1)

    def set_position(self, pos: int) -> None:
        """The position of the next token fed (the cache length before it)."""
        self.pos64.fill_(pos)
        self.pos32.fill_(pos)
        self.len32.fill_(pos + 1)
        self._host_pos = pos

    @torch.no_grad()
    def step(self) -> None:
        if self._host_pos is None or self._host_pos >= self.max_len:
            raise _lib.LeanKVError("BatchedEngine: position %s outside the cache's %d tokens"
                                   % (self._host_pos, self.max_len))
        if self.graph is None:
            self._step()  # eager: allocates what the step needs, then capture
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                with torch.cuda.graph(g, stream=s):
                    self._step()
            torch.cuda.current_stream().wait_stream(s)
            self.graph = g
        else:
            self.graph.replay()
        self._host_pos += 1


class GenerateFastPath:
    """model.forward for HF ``generate``: single-token decode steps on graph-replayed decode engines.

    The reference's user path is ``model.generate(..., past_key_values=cache)``
    (leankv/combined.py:13, scripts/benchmark.py:68-99), whose decode steps walk
    the HF modules in Python, one patched projection at a time.  Installed on a
    TEAL-patched model, this wrapper sends a call that LeanKVEngine computes the
    same way -- one new token of one sequence (input_ids [1, 1]), a fused
    TurboQuantCache at 1 to 4 bits with a window of at most 256 tokens, no padding, no sliding
    window shorter than the sequence, no attentions or hidden states asked for
    -- to the engine, built on that cache's own buffers and replayed as a HIP
    graph; it appends the token to the cache as update() would and returns the
    last position's logits.  A step of B > 1 sequences of one length (no
    padding) on a fused cache goes to BatchedEngine, the HF forward's own
    sequence of calls replayed as a graph (equal logits).  Every other call
    (the prefill, padded batches, other caches) runs the model's own forward.
    ``steps`` counts the calls served each way."""

    def __init__(self, model):
        import inspect

        self.model = model
        self.forward = model.forward  # the model's own forward (bound)
        # generate inspects forward's parameters (logits_to_keep, ...): report the model's own
        self.__signature__ = inspect.signature(self.forward)
        self.engine = None
        self._cache = None  # the cache the B = 1 engine was built on
        self.batched = None  # BatchedEngine for B > 1 calls
        self._engine_key = None   # (cache, its storage generation, length bound) the engines were built for
        self._batched_key = None
        self._model_why = False   # not asked yet; then None (the engines can run the model) or the reason
        self._model_why_key = None  # the model state the answer was given for (_model_state)
        self._step_why = {}       # cache geometry -> None or why lkv_decode_* refuses it
        self.steps = {"engine": 0, "batch": 0, "forward": 0}

    def _eligible(self, input_ids, cache, kw) -> str | None:
        """"one" (the fused B=1 step), "batch" (BatchedEngine) or None (the model's forward)."""
        if not isinstance(cache, TurboQuantCache) or not cache.fused_attention or not cache.fused_decode:
            return None
        if input_ids is None or input_ids.dim() != 2 or input_ids.shape[1] != 1:
            return None
        if kw.get("inputs_embeds") is not None or kw.get("output_attentions") or kw.get("output_hidden_states"):
            return None
        if kw.get("return_dict") is False or kw.get("use_cache") is False or kw.get("labels") is not None:
            return None
        B = input_ids.shape[0]
        if cache.head_dim != 128 or cache._k_codes[0] is None or cache._k_codes[0].shape[0] != B:
            return None
        if self._model_reason() is not None:
            return None
        if B == 1 and self._step_reason(cache) is not None:
            return None
        n = cache._seq_lengths[0]
        if n == 0 or any(x != n for x in cache._seq_lengths) or any(cache._fused_pending) or \
                any(cache._prefill_pending):
            return None
        if n + 1 > cache.attn_max_len(0):  # the append would grow the store: the forward does that
            return None
        sw = getattr(self.model.config, "sliding_window", None)
        if sw is not None and sw <= n:
            return None
        mask = kw.get("attention_mask")
        if mask is not None and (mask.shape[-1] != n + 1 or not bool(mask.all())):
            return None
        return "one" if B == 1 else "batch"

    def _model_reason(self) -> str | None:
        """Why neither engine can run this model (None if both can): the fused kernels read fp16 weights,
        norms and embeddings through raw pointers and have no projection bias, so a model in another dtype or
        with a bias stays on its own forward (which raises or runs as it would without this wrapper)."""
        state = self._model_state()
        if self._model_why is not False and self._model_why_key == state:
            return self._model_why
        why = None
        m = self.model
        cfg = m.config
        D = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        if D != 128:
            why = "head_dim %d (the kernels take 128)" % D
        tensors = [("embed_tokens", m.model.embed_tokens.weight), ("norm", m.model.norm.weight),
                   ("lm_head", m.lm_head.weight)]
        for i, layer in enumerate(m.model.layers):
            tensors += [("layers.%d.input_layernorm" % i, layer.input_layernorm.weight),
                        ("layers.%d.post_attention_layernorm" % i, layer.post_attention_layernorm.weight)]
            for name, mod in (("q_proj", layer.self_attn.q_proj), ("k_proj", layer.self_attn.k_proj),
                              ("v_proj", layer.self_attn.v_proj), ("o_proj", layer.self_attn.o_proj),
                              ("gate_proj", layer.mlp.gate_proj), ("up_proj", layer.mlp.up_proj),
                              ("down_proj", layer.mlp.down_proj)):
                tensors.append(("layers.%d.%s" % (i, name), mod.weight))
                if why is None and getattr(mod, "bias", None) is not None:
                    why = "layers.%d.%s has a bias" % (i, name)
        for name, t in tensors:
            if why is None and t.dtype != torch.float16:
                why = "%s is %s (the fused kernels read fp16)" % (name, t.dtype)
        self._model_why = why
        self._model_why_key = state
        return why

    def _model_state(self) -> tuple:
        """Identity of the tensors the engines hold raw pointers to, cheap enough to take per call: a model
        moved to another dtype or device (model.half(), model.to(...)) replaces its embedding and lm_head
        storage, so the eligibility is asked again and the engines are rebuilt."""
        e, h = self.model.model.embed_tokens.weight, self.model.lm_head.weight
        return (e.dtype, e.data_ptr(), h.dtype, h.data_ptr())

    def _step_reason(self, cache: TurboQuantCache) -> str | None:
        """Why the fused B = 1 step (lkv_decode_*) cannot run this model on this cache (None if it can): the
        library's own shape check on the step's dimensions, asked once per cache geometry."""
        key = (cache.bits, cache.hot_buffer_size, cache.cold_capacity(0))
        if key in self._step_why:
            return self._step_why[key]
        cfg = self.model.config
        why = None
        if cache.bits not in STEP_BITS:
            why = "bits=%d (the fused step takes %s)" % (cache.bits, STEP_BITS)
        else:
            # validation only: check_dims tests the pointers for null and alignment, never dereferences them
            fake = 256
            dims = _lib.DecodeDims(
                hidden=cfg.hidden_size, ffn=cfg.intermediate_size, vocab=cfg.vocab_size,
                n_heads=cfg.num_attention_heads, n_kv_heads=cfg.num_key_value_heads,
                max_len=cache.attn_max_len(0), cap=cache.cold_capacity(0), hot_cap=cache.hot_buffer_size,
                bits=cache.bits, eps=float(cfg.rms_norm_eps), scale=1.0 / math.sqrt(128.0),
                bounds=fake, centroids=fake, rope_cos=fake, rope_sin=fake)
            if _lib.load().lkv_decode_workspace_bytes(ctypes.byref(dims)) == 0:
                why = _lib.last_error()
        self._step_why[key] = why
        return why

    def _engine_for(self, cache: TurboQuantCache) -> "LeanKVEngine":
        # the engine holds raw pointers to the cache's buffers (and its graph captured them): buffers that
        # were replaced since -- a store that grew, a reset() followed by a new prefill -- need a new engine
        key = (id(cache), cache.storage_generation, cache.attn_max_len(0), self._model_state())
        if self.engine is not None and self._cache is cache and self._engine_key == key:
            return self.engine
        self.engine = None
        torch.cuda.empty_cache()
        self.engine = LeanKVEngine(self.model, cache, cache.attn_max_len(0))
        self._cache = cache
        self._engine_key = key
        return self.engine

    def _batched_for(self, cache: TurboQuantCache, B: int) -> BatchedEngine:
        key = (id(cache), cache.storage_generation, cache.attn_max_len(0), B, self._model_state())
        be = self.batched
        if be is None or be.cache is not cache or self._batched_key != key:
            self.batched = None
            torch.cuda.empty_cache()
            self.batched = BatchedEngine(self.model, cache, B)
            self._batched_key = key
        return self.batched

    def __call__(self, input_ids=None, *args, **kw):
        cache = kw.get("past_key_values")
        kind = None if args else self._eligible(input_ids, cache, kw)
        if kind is None:
            self.steps["forward"] += 1
            return self.forward(input_ids, *args, **kw)
        from transformers.modeling_outputs import CausalLMOutputWithPast

        n = cache._seq_lengths[0]
        if kind == "batch":
            be = self._batched_for(cache, input_ids.shape[0])
            with torch.no_grad():
                if be._host_pos != n:
                    be.set_position(n)
                be.tok.copy_(input_ids.view(-1))
                be.step()
                cache._seen_tokens += 1
                for li in range(cache.num_layers):
                    cache._seq_lengths[li] = n + 1
                logits = be.logits.clone()
            self.steps["batch"] += 1
            return CausalLMOutputWithPast(logits=logits, past_key_values=cache)
        eng = self._engine_for(cache)
        with torch.no_grad():
            if eng._host_pos != n:
                eng._set_start(input_ids.view(1), n)
            else:
                eng.tok.copy_(input_ids.view(1))
            first = eng.graph is None
            eng.step()
            if first:
                eng.capture()
            # the step appended the token to every layer (ring slot, the evicted token's codes): the
            # cache's counters follow, as update() would have moved them
            cache._seen_tokens += 1
            for li in range(cache.num_layers):
                cache._seq_lengths[li] = n + 1
            logits = eng.logits.view(1, 1, -1).clone()
        self.steps["engine"] += 1
        return CausalLMOutputWithPast(logits=logits, past_key_values=cache)


def enable_generate_fast_path(model) -> GenerateFastPath:
    """Install GenerateFastPath as model.forward (idempotent); every projection must be TEAL-patched, so the
    engine reads the patched column-major weights instead of copying them."""
    if isinstance(getattr(model, "forward", None), GenerateFastPath):
        return model.forward
    for layer in model.model.layers:
        for mod in (layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj, layer.self_attn.o_proj,
                    layer.mlp.gate_proj, layer.mlp.up_proj, layer.mlp.down_proj):
            if getattr(mod, "_teal_threshold", None) is None:
                raise ValueError("enable_generate_fast_path: every projection must be TEAL-patched first")
    fp = GenerateFastPath(model)
    model.forward = fp
    return fp


def disable_generate_fast_path(model) -> None:
    fp = getattr(model, "forward", None)
    if isinstance(fp, GenerateFastPath):
        model.forward = fp.forward
        fp.engine = None
        fp.batched = None


class OwnDenseEngine(_Base):
    """Dense fp16 decode on this library's kernels: the dense baseline of the LeanKV engine.

    The reference's baseline is plain HF decode with fp16 weights and an fp16 KV
    cache (scripts/raw_baseline.py:33-62).  Here it is the fused decode step of
    LeanKVEngine with every TEAL threshold 0 (the GEMVs read every weight row)
    and an fp16 KV cache in 16-token pages (lkv_decode_layer_step_f16kv: the
    step's key and value go to the pool, lkv_paged_decode_attn attends), so the
    two engines differ only in TEAL and TurboQuant.  Weights are read
    column-major; ones that are not get a column-major copy.  Graph-captured
    like LeanKVEngine.
    """

    PAGE = 16  # tokens per page of the fp16 pool (lkv_decode_layer_step_f16kv)

    def __init__(self, model, max_len: int):
        super().__init__(model, max_len)
        if self.D != 128:
            raise ValueError("the fused decode step needs head_dim 128, got %d" % self.D)
        from .turboquant.codebook import get_codebook_tensors

        lib = _lib.load()
        d = self.dev
        self._keep = []
        cent, bnd = get_codebook_tensors(128, 3, d, torch.float32)  # validated by the step, not used by it
        self.dims = _lib.DecodeDims(
            hidden=self.hidden, ffn=self.cfg.intermediate_size, vocab=self.cfg.vocab_size, n_heads=self.H,
            n_kv_heads=self.Hkv, max_len=max_len, cap=max_len, hot_cap=64, bits=3, eps=self.eps, scale=self.scale,
            bounds=self._hold(bnd[1:-1].contiguous()), centroids=self._hold(cent.contiguous()),
            rope_cos=self._hold(self.cos), rope_sin=self._hold(self.sin))
        self.pages = (max_len + self.PAGE - 1) // self.PAGE
        self.pools = [torch.zeros(self.pages, 2, self.PAGE, self.Hkv, self.D, dtype=torch.float16, device=d)
                      for _ in range(self.L)]
        self.layer_structs = []
        for layer in self.layers:
            at, mlp = layer.self_attn, layer.mlp
            w = {}
            for name, mod in (("q", at.q_proj), ("k", at.k_proj), ("v", at.v_proj), ("o", at.o_proj),
                              ("g", mlp.gate_proj), ("u", mlp.up_proj), ("d", mlp.down_proj)):
                if getattr(mod, "bias", None) is not None:
                    raise ValueError("the fused decode step has no projection bias")
                w[name] = self._hold(_colmajor(mod.weight))
            self.layer_structs.append(_lib.DecodeLayer(
                input_norm=self._hold(layer.input_layernorm.weight.detach()),
                post_norm=self._hold(layer.post_attention_layernorm.weight.detach()),
                wq=w["q"], wk=w["k"], wv=w["v"], wo=w["o"], wg=w["g"], wu=w["u"], wd=w["d"],
                tq=0.0, tk=0.0, tv=0.0, to=0.0, tg=0.0, tu=0.0, td=0.0))
        self.final_norm = model.model.norm.weight.detach()
        self.lm_head_cm = model.lm_head.weight.detach().t().contiguous()
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

    def load_cache(self, past_key_values) -> int:
        """Copy a prefilled HF DynamicCache (K/V [1, Hkv, n, 128]) into the page pools; returns its length."""
        n = 0
        for i in range(self.L):
            lay = past_key_values.layers[i]
            for half, t in ((0, lay.keys), (1, lay.values)):
                n = t.shape[2]
                if n > self.max_len:
                    raise _lib.LeanKVError("prefilled cache of %d tokens exceeds max_len %d" % (n, self.max_len))
                rows = t[0].transpose(0, 1)  # [n, Hkv, 128]
                full, rest = divmod(n, self.PAGE)
                if full:
                    self.pools[i][:full, half] = rows[: full * self.PAGE].reshape(full, self.PAGE, self.Hkv, self.D)
                if rest:
                    self.pools[i][full, half, :rest] = rows[full * self.PAGE:]
        return n

    def start(self, first_token: torch.Tensor, length: int) -> None:
        self._set_start(first_token, length)

    def _step(self) -> None:
        lib = _lib.load()
        st = _lib.stream_handle(self.dev)
        ws, nb = self.ws.data_ptr(), self.ws.numel()
        dims = ctypes.byref(self.dims)
        _lib.check(lib.lkv_decode_begin(dims, self.model.model.embed_tokens.weight.data_ptr(), self.tok.data_ptr(),
                                        self.pos64.data_ptr(), self.x.data_ptr(), ws, nb, st), "lkv_decode_begin")
        for ls, pool in zip(self.layer_structs, self.pools):
            _lib.check(lib.lkv_decode_layer_step_f16kv(dims, ctypes.byref(ls), pool.data_ptr(), self.x.data_ptr(),
                                                       ws, nb, st), "lkv_decode_layer_step_f16kv")
        _lib.check(lib.lkv_decode_head(dims, self.final_norm.data_ptr(), self.lm_head_cm.data_ptr(),
                                       self.x.data_ptr(), self.logits.data_ptr(), self.tok.data_ptr(),
                                       self.pos64.data_ptr(), self.hist.data_ptr(), self.hist.numel(), ws, nb, st),
                   "lkv_decode_head")


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
        self._set_start(first_token, length)

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


# Mistral-7B-v0.3 shape (the config-5 decoder; configs/mistral7b.yaml in the reference).
# Mistral-7B-v0.3 has no sliding window ("sliding_window": null); MistralConfig's default is 4096.
MISTRAL_7B = dict(vocab_size=32768, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                  num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=32768,
                  rope_theta=1e6, rms_norm_eps=1e-5, sliding_window=None)


# Llama-3-8B (named beside Mistral-7B by the reference's docs): the same decoder with a 128 K
# vocabulary and RoPE base 500000.  Llama-3.1's "llama3" frequency scaling is an override:
# rope_scaling=LLAMA31_ROPE, max_position_embeddings=131072.
LLAMA3_8B = dict(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                 num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=8192,
                 rope_theta=500000.0, rms_norm_eps=1e-5)
LLAMA31_ROPE = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                "original_max_position_embeddings": 8192}


@torch.no_grad()
def random_llama(device="cuda", seed: int = 0, **overrides):
    """Random-init fp16 LlamaForCausalLM of the Llama-3-8B shape (overridable), built as random_mistral."""
    from transformers import LlamaConfig, LlamaForCausalLM

    kw = dict(LLAMA3_8B)
    kw.update(overrides)
    return _random_init(LlamaForCausalLM, LlamaConfig(**kw), device, seed)


def _random_init(cls, cfg, device, seed):
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device(device):
            model = cls(cfg)
    finally:
        torch.set_default_dtype(prev)
    gen = torch.Generator(device=device).manual_seed(seed)
    for name, p in model.named_parameters():
        if p.dim() == 2:
            p.copy_(torch.randn(p.shape, generator=gen, device=device, dtype=torch.float32).mul_(0.02).to(p.dtype))
        else:
            p.fill_(1.0)
    model.eval()
    return model


@torch.no_grad()
def random_mistral(device="cuda", seed: int = 0, **overrides):
    """Random-init fp16 MistralForCausalLM (weights ~N(0, 0.02), norms 1) built directly on `device`.

    The model is constructed with fp16 as the default dtype, as from_pretrained(torch_dtype=float16) does:
    parameters are fp16 while the rotary embedding keeps its fp32 inverse frequencies (a ``.to(float16)``
    of the whole module would round them to fp16 and shift RoPE angles by ~position * 2^-11 rad)."""
    from transformers import MistralConfig, MistralForCausalLM

    kw = dict(MISTRAL_7B)
    kw.update(overrides)
    return _random_init(MistralForCausalLM, MistralConfig(**kw), device, seed)
