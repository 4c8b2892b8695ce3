"""Greedy decoding of a Gemma-2 decoder with a static KV cache, built so that
one decode step (one new token per sequence) is captured in a HIP graph and
replayed back to back: the end-to-end tokens/s then measures the kernels,
not the Python above them.

The architecture follows transformers' Gemma2 (modeling_gemma2.py):
RMSNorm x * rsqrt(mean(x^2) + eps) * (1 + w) in FP32; embedding rows times
sqrt(hidden) in BF16; grouped-query attention with RoPE, scaling
query_pre_attn_scalar^-1/2, logit soft-capping tanh(s/50)*50 and a sliding
window on even layers; gelu(tanh) gated MLP; post-attention and
post-feed-forward norms; tied LM head with final soft-capping tanh(z/30)*30.

The linear layers come from one of three backends with the same call
pattern (q/k/v and gate/up issued as one grouped product each):
  "se12" - the fused SE12 kernels for decode steps; prefill decodes each
           layer into a shared scratch buffer and runs F.linear (exact);
  "raw"  - the raw-BF16 twin kernels for decode steps, F.linear for prefill:
           with the same launch shapes it gives the "se12" logits bit for bit;
  "bf16" - hipBLASLt through F.linear for everything (concatenated q/k/v and
           gate/up weights).
Batched products whose right operand is a transposed view are avoided (the
K cache is kept transposed and contiguous): they have faulted MI355X GPUs.

A decode step runs either through the library's step kernels (include/
se12_step.h: fused norms, attention, activation, logits; the default, ~8
launches per layer) or through framework ops (`fused_step=False`, ~80 small
kernels per layer; kept as the reference the step kernels are tested
against).
"""

from __future__ import annotations

import dataclasses
import math

import torch
import torch.nn.functional as F

from . import _native as nat


@dataclasses.dataclass(frozen=True)
class Gemma2Shape:
    layers: int = 26
    hidden: int = 2304
    intermediate: int = 9216
    heads: int = 8
    kv_heads: int = 4
    head_dim: int = 256
    vocab: int = 256000
    eps: float = 1e-6
    rope_theta: float = 10000.0
    query_pre_attn_scalar: float = 256.0
    attn_softcap: float = 50.0
    final_softcap: float = 30.0
    sliding_window: int = 4096


GEMMA2_2B = Gemma2Shape()
PROJECTIONS = ("q", "k", "v", "o", "gate", "up", "down")


def projection_shapes(s: Gemma2Shape) -> dict[str, tuple[int, int]]:
    return {"q": (s.heads * s.head_dim, s.hidden), "k": (s.kv_heads * s.head_dim, s.hidden),
            "v": (s.kv_heads * s.head_dim, s.hidden), "o": (s.hidden, s.heads * s.head_dim),
            "gate": (s.intermediate, s.hidden), "up": (s.intermediate, s.hidden), "down": (s.hidden, s.intermediate)}


@dataclasses.dataclass
class Gemma2Weights:
    """BF16 weights on the device: per layer the 7 projections and 4 norm
    weights, the tied embedding and the final norm."""

    shape: Gemma2Shape
    layers: list[dict[str, torch.Tensor]]
    embed: torch.Tensor
    final_norm: torch.Tensor

    @classmethod
    def random(cls, shape: Gemma2Shape, device, std: float = 0.02, seed: int = 0) -> "Gemma2Weights":
        """BF16 N(0, std) projections and embedding, seeded per tensor; norm
        weights zero (transformers' Gemma2 initialisation)."""
        gen = torch.Generator(device=device)
        shapes = projection_shapes(shape)
        layers = []
        for li in range(shape.layers):
            lw = {}
            for pi, name in enumerate(PROJECTIONS):
                gen.manual_seed(seed * 1_000_003 + li * 100 + pi)
                lw[name] = (torch.randn(shapes[name], generator=gen, device=device) * std).to(torch.bfloat16)
            for nm in ("input_norm", "post_attn_norm", "pre_ffw_norm", "post_ffw_norm"):
                lw[nm] = torch.zeros(shape.hidden, dtype=torch.bfloat16, device=device)
            layers.append(lw)
        gen.manual_seed(seed * 1_000_003 + 99_999)
        embed = (torch.randn((shape.vocab, shape.hidden), generator=gen, device=device) * std).to(torch.bfloat16)
        return cls(shape, layers, embed, torch.zeros(shape.hidden, dtype=torch.bfloat16, device=device))

    @classmethod
    def from_hf(cls, model) -> "Gemma2Weights":
        """The weights of a transformers Gemma2ForCausalLM with nn.Linear layers."""
        c = model.config
        shape = Gemma2Shape(layers=c.num_hidden_layers, hidden=c.hidden_size, intermediate=c.intermediate_size,
                            heads=c.num_attention_heads, kv_heads=c.num_key_value_heads, head_dim=c.head_dim,
                            vocab=c.vocab_size, eps=c.rms_norm_eps, rope_theta=c.rope_parameters["rope_theta"],
                            query_pre_attn_scalar=c.query_pre_attn_scalar, attn_softcap=c.attn_logit_softcapping,
                            final_softcap=c.final_logit_softcapping, sliding_window=c.sliding_window)
        layers = []
        for layer in model.model.layers:
            a, m = layer.self_attn, layer.mlp
            layers.append({"q": a.q_proj.weight.data, "k": a.k_proj.weight.data, "v": a.v_proj.weight.data,
                           "o": a.o_proj.weight.data, "gate": m.gate_proj.weight.data, "up": m.up_proj.weight.data,
                           "down": m.down_proj.weight.data, "input_norm": layer.input_layernorm.weight.data,
                           "post_attn_norm": layer.post_attention_layernorm.weight.data,
                           "pre_ffw_norm": layer.pre_feedforward_layernorm.weight.data,
                           "post_ffw_norm": layer.post_feedforward_layernorm.weight.data})
        return cls(shape, layers, model.model.embed_tokens.weight.data, model.model.norm.weight.data)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    out = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (out * (1.0 + w.float())).type_as(x)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class _Backend:
    """Linear layers of the whole stack for one backend."""

    def __init__(self, kind: str, w: Gemma2Weights, max_batch: int, scratch: torch.Tensor | None = None,
                 encoded: dict | None = None) -> None:
        from .hip import RawBf16MatVecKernel, Se12MatVecKernel

        self.kind = kind
        self.w = w
        self.layers = []
        if kind == "se12":
            biggest = max(max(t.numel() for n, t in lw.items() if n in PROJECTIONS) for lw in w.layers)
            self.scratch = scratch if scratch is not None else torch.empty(
                biggest, dtype=torch.bfloat16, device=w.embed.device)
        for li, lw in enumerate(w.layers):
            if kind == "se12":
                ks = {n: Se12MatVecKernel(encoded[(li, n)], max_batch=max_batch) for n in PROJECTIONS}
            elif kind == "raw":
                ks = {n: RawBf16MatVecKernel(lw[n], max_batch=max_batch) for n in PROJECTIONS}
            elif kind == "bf16":
                ks = {"qkv": torch.cat([lw["q"], lw["k"], lw["v"]]), "gate_up": torch.cat([lw["gate"], lw["up"]])}
            else:
                raise ValueError(f"unknown backend {kind!r}")
            self.layers.append(ks)
        if kind == "se12":
            self.lm_head = Se12MatVecKernel(encoded["embed"], max_batch=max_batch)
        elif kind == "raw":
            self.lm_head = RawBf16MatVecKernel(w.embed, max_batch=max_batch)

    # -- prefill: exact products --------------------------------------------
    def prefill_weight(self, li: int, name: str) -> torch.Tensor:
        if self.kind == "se12":
            k = self.layers[li][name]
            return k.decode_into(self.scratch[: k.rows * k.cols].view(k.rows, k.cols))
        return self.w.layers[li][name]

    # -- decode steps -------------------------------------------------------
    def grouped(self, li: int, names: tuple[str, ...], x: torch.Tensor) -> list[torch.Tensor]:
        if self.kind == "bf16":
            y = F.linear(x, self.layers[li]["qkv" if names[0] == "q" else "gate_up"])
            sizes = [self.w.layers[li][n].shape[0] for n in names]
            return list(torch.split(y, sizes, dim=-1))
        from .hip import multiply_grouped

        return [y.to(torch.bfloat16) for y in multiply_grouped([self.layers[li][n] for n in names], x)]

    def single(self, li: int, name: str, x: torch.Tensor) -> torch.Tensor:
        if self.kind == "bf16":
            return F.linear(x, self.w.layers[li][name])
        return self.layers[li][name].multiply(x).to(torch.bfloat16)

    def logits(self, x: torch.Tensor) -> torch.Tensor:
        if self.kind == "bf16":
            return F.linear(x, self.w.embed)
        return self.lm_head.multiply(x).to(torch.bfloat16)

    # -- fused decode steps: raw products (FP32 for the library kernels, BF16
    # for hipBLASLt), consumed by the step kernels ---------------------------
    def grouped_raw(self, li: int, names: tuple[str, ...], x: torch.Tensor, outs: list[torch.Tensor] | None):
        """[(tensor, column offset, row stride)] per name."""
        if self.kind == "bf16":
            y = F.linear(x, self.layers[li]["qkv" if names[0] == "q" else "gate_up"])
            offs, res = 0, []
            for n in names:
                res.append((y, offs, y.shape[1]))
                offs += self.w.layers[li][n].shape[0]
            return res
        from .hip import multiply_grouped

        ys = multiply_grouped([self.layers[li][n] for n in names], x, outs=outs)
        return [(y, 0, y.shape[1]) for y in ys]

    def single_raw(self, li: int, name: str, x: torch.Tensor, out: torch.Tensor | None) -> torch.Tensor:
        if self.kind == "bf16":
            return F.linear(x, self.w.layers[li][name])
        return self.layers[li][name].multiply(x, out=out)

    def logits_raw(self, x: torch.Tensor, out: torch.Tensor | None) -> torch.Tensor:
        if self.kind == "bf16":
            return F.linear(x, self.w.embed)
        return self.lm_head.multiply(x, out=out)

    def embed_into(self, ids: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        if self.kind == "se12":
            return self.lm_head.decode_rows_into(ids.reshape(-1), out)
        return torch.index_select(self.w.embed, 0, ids.reshape(-1), out=out)

    def embed_rows(self, ids: torch.Tensor) -> torch.Tensor:
        if self.kind == "se12":
            out = torch.empty((ids.numel(), self.w.shape.hidden), dtype=torch.bfloat16, device=ids.device)
            return self.lm_head.decode_rows_into(ids.reshape(-1), out)
        return self.w.embed[ids.reshape(-1)]


class Gemma2Decoder:
    """Prefill + graph-captured greedy decode over one backend."""

    def __init__(self, weights: Gemma2Weights, backend: str, batch: int, max_len: int,
                 encoded: dict | None = None, max_batch: int = nat.MAX_BATCH, scratch: torch.Tensor | None = None,
                 fused_step: bool = True, fused_tails: bool = True):
        s = weights.shape
        max_len = -(-max_len // 8) * 8          # the step kernels read the caches 8 positions at a time
        self.s, self.w, self.batch, self.max_len = s, weights, batch, max_len
        dev = weights.embed.device
        self.dev = dev
        self.be = _Backend(backend, weights, max_batch, scratch=scratch, encoded=encoded)
        self.kt = [torch.zeros((batch, s.kv_heads, s.head_dim, max_len), dtype=torch.bfloat16, device=dev)
                   for _ in range(s.layers)]
        self.v = [torch.zeros((batch, s.kv_heads, max_len, s.head_dim), dtype=torch.bfloat16, device=dev)
                  for _ in range(s.layers)]
        self.inv_freq = 1.0 / (s.rope_theta ** (torch.arange(0, s.head_dim, 2, dtype=torch.int64, device=dev).float() / s.head_dim))
        self.scaling = s.query_pre_attn_scalar ** -0.5
        self.embed_scale = torch.tensor(math.sqrt(s.hidden), dtype=torch.bfloat16, device=dev)
        self.ids = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.pos = torch.zeros((), dtype=torch.int64, device=dev)
        self.step_index = torch.zeros((), dtype=torch.int64, device=dev)
        self.tokens = torch.zeros((batch, max_len), dtype=torch.int64, device=dev)
        self.last_logits = torch.zeros((batch, s.vocab), dtype=torch.bfloat16, device=dev)
        self.graph = None
        self.fused_step = fused_step
        # the library backends run the MLP gate and the residual norms in the
        # tails of the products that feed them (se12_gemv_gelu_mul / _rmsnorm)
        self.fused_tails = fused_step and fused_tails and backend != "bf16"
        if fused_step:
            f32 = backend != "bf16"
            shapes = projection_shapes(s)

            def buf(n, dtype=torch.float32):
                return torch.empty((batch, n), dtype=dtype, device=dev)

            self.x = buf(s.hidden, torch.bfloat16)          # residual stream
            # the products with the norm in their head write the updated
            # residual to the other buffer; `residual` is the current one
            # after a step
            self.x2 = buf(s.hidden, torch.bfloat16) if self.fused_tails else None
            # tile-row sums of squares of o_proj's and down_proj's outputs,
            # written by those products for the norms in the next heads
            self.o_ss = buf((s.hidden + 15) // 16, torch.float32) if self.fused_tails else None
            self.down_ss = buf((s.hidden + 15) // 16, torch.float32) if self.fused_tails else None
            self.residual = self.x
            self.h = buf(s.hidden, torch.bfloat16)          # normalised input of the next product
            self.emb = buf(s.hidden, torch.bfloat16)
            self.attn = buf(s.heads * s.head_dim, torch.bfloat16)
            self.m = buf(s.intermediate, torch.bfloat16)
            self.qkv = [buf(shapes[n][0]) for n in ("q", "k", "v")] if f32 else None
            self.gu = [buf(s.intermediate), buf(s.intermediate)] if f32 else None
            self.o_out = buf(s.hidden) if f32 else None
            self.down_out = buf(s.hidden) if f32 else None
            self.logits_out = buf(s.vocab) if f32 else None
            self.embed_scale_value = float(self.embed_scale.float().item())
            n = nat.lib().se12_step_attention_workspace(batch, s.heads, s.kv_heads, s.head_dim, max_len)
            if n < 0:
                nat.step_check(n)
            self.attn_ws = torch.zeros(n, dtype=torch.uint8, device=dev)   # counters start at zero
            n = nat.lib().se12_step_logits_workspace(batch, s.vocab)
            if n < 0:
                nat.step_check(n)
            self.logits_ws = torch.zeros(n, dtype=torch.uint8, device=dev)

    def _rope(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        freqs = positions.float()[..., None] * self.inv_freq
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)

    def _finish(self, x: torch.Tensor) -> torch.Tensor:
        s = self.s
        x = rms_norm(x, self.w.final_norm, s.eps)
        logits = self.be.logits(x)
        return torch.tanh(logits / s.final_softcap) * s.final_softcap

    # -- prefill ------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        """Runs the prompt [batch, T] (exact products), fills the KV cache and
        returns the first generated token per sequence."""
        s, B = self.s, self.batch
        T = prompt.shape[1]
        x = (self.be.embed_rows(prompt) * self.embed_scale).view(B, T, s.hidden)
        cos, sin = self._rope(torch.arange(T, device=self.dev))
        i = torch.arange(T, device=self.dev)
        causal = i[None, :] <= i[:, None]
        for li, lw in enumerate(self.w.layers):
            h = rms_norm(x, lw["input_norm"], s.eps)
            q = F.linear(h, self.be.prefill_weight(li, "q")).view(B, T, s.heads, s.head_dim).transpose(1, 2)
            k = F.linear(h, self.be.prefill_weight(li, "k")).view(B, T, s.kv_heads, s.head_dim).transpose(1, 2)
            v = F.linear(h, self.be.prefill_weight(li, "v")).view(B, T, s.kv_heads, s.head_dim).transpose(1, 2)
            q = q * cos + rotate_half(q) * sin
            k = k * cos + rotate_half(k) * sin
            self.kt[li][:, :, :, :T] = k.transpose(2, 3)
            self.v[li][:, :, :T, :] = v
            g = s.heads // s.kv_heads
            kt = k.transpose(2, 3).contiguous()                       # [B, kvh, d, T]
            qg = q.reshape(B, s.kv_heads, g * T, s.head_dim)           # heads grouped by kv head
            sc = torch.matmul(qg, kt).view(B, s.kv_heads, g, T, T) * self.scaling
            sc = torch.tanh(sc / s.attn_softcap) * s.attn_softcap
            allowed = causal if li % 2 else causal & (i[:, None] - i[None, :] < s.sliding_window)
            sc = sc.masked_fill(~allowed, float("-inf"))
            p = F.softmax(sc.float(), dim=-1).to(torch.bfloat16).view(B, s.kv_heads, g * T, T)
            o = torch.matmul(p, v.contiguous()).view(B, s.heads, T, s.head_dim).transpose(1, 2).reshape(B, T, -1)
            o = F.linear(o, self.be.prefill_weight(li, "o"))
            x = x + rms_norm(o, lw["post_attn_norm"], s.eps)
            h = rms_norm(x, lw["pre_ffw_norm"], s.eps)
            mm = F.gelu(F.linear(h, self.be.prefill_weight(li, "gate")), approximate="tanh") * \
                F.linear(h, self.be.prefill_weight(li, "up"))
            x = x + rms_norm(F.linear(mm, self.be.prefill_weight(li, "down")), lw["post_ffw_norm"], s.eps)
        logits = self._finish(x[:, -1, :].contiguous())
        self.last_logits.copy_(logits)
        first = logits.argmax(-1)
        self.ids.copy_(first)
        self.pos.fill_(T)
        self.tokens.zero_()
        self.tokens[:, 0] = first
        self.step_index.fill_(1)
        return first

    # -- one decode step (captured) -----------------------------------------
    def _step(self) -> None:
        s, B = self.s, self.batch
        x = self.be.embed_rows(self.ids) * self.embed_scale                         # [B, H]
        cos, sin = self._rope(self.pos.view(1))
        j = torch.arange(self.max_len, device=self.dev)
        past = j <= self.pos
        window = past & (self.pos - j < s.sliding_window)
        g = s.heads // s.kv_heads
        for li, lw in enumerate(self.w.layers):
            h = rms_norm(x, lw["input_norm"], s.eps)
            q, k, v = self.be.grouped(li, ("q", "k", "v"), h)
            q = q.view(B, s.heads, s.head_dim)
            k = k.view(B, s.kv_heads, s.head_dim)
            q = q * cos + rotate_half(q) * sin
            k = k * cos + rotate_half(k) * sin
            self.kt[li].index_copy_(3, self.pos.view(1), k.unsqueeze(-1))
            self.v[li].index_copy_(2, self.pos.view(1), v.view(B, s.kv_heads, 1, s.head_dim))
            sc = torch.matmul(q.view(B, s.kv_heads, g, s.head_dim), self.kt[li]) * self.scaling   # [B, kvh, g, L]
            sc = torch.tanh(sc / s.attn_softcap) * s.attn_softcap
            sc = sc.masked_fill(~(past if li % 2 else window), float("-inf"))
            p = F.softmax(sc.float(), dim=-1).to(torch.bfloat16)
            o = torch.matmul(p, self.v[li]).reshape(B, s.heads * s.head_dim)
            o = self.be.single(li, "o", o)
            x = x + rms_norm(o, lw["post_attn_norm"], s.eps)
            h = rms_norm(x, lw["pre_ffw_norm"], s.eps)
            gt, up = self.be.grouped(li, ("gate", "up"), h)
            x = x + rms_norm(self.be.single(li, "down", F.gelu(gt, approximate="tanh") * up), lw["post_ffw_norm"], s.eps)
        logits = self._finish(x)
        self.last_logits.copy_(logits)
        nxt = logits.argmax(-1)
        self.ids.copy_(nxt)
        self.tokens.index_copy_(1, self.step_index.view(1), nxt.view(B, 1))
        self.pos.add_(1)
        self.step_index.add_(1)

    # -- one decode step through the step kernels (captured) ------------------
    def _step_fused(self) -> None:
        s, B = self.s, self.batch
        lib = nat.lib()
        st = nat.stream_ptr()
        BF16, F32 = nat.STEP_BF16, nat.STEP_F32
        ck = nat.step_check

        def dt(t: torch.Tensor) -> int:
            return F32 if t.dtype == torch.float32 else BF16

        def at(t: torch.Tensor, col: int) -> int:
            return t.data_ptr() + col * t.element_size()

        self.be.embed_into(self.ids, self.emb)
        ck(lib.se12_step_rmsnorm(nat.ptr(self.emb), BF16, s.hidden, nat.ptr(self.w.layers[0]["input_norm"]),
                                 nat.ptr(self.x), None, nat.ptr(self.h), B, s.hidden, s.eps, self.embed_scale_value, 0, st))
        if self.fused_tails:
            self._layers_fused_tails()
        else:
            for li, lw in enumerate(self.w.layers):
                (q, qo, qs), (k, ko, ks), (v, vo, _) = self.be.grouped_raw(li, ("q", "k", "v"), self.h, self.qkv)
                self._attention(li, at(q, qo), at(k, ko), at(v, vo), dt(q), qs, ks)
                nxt = self.w.layers[li + 1]["input_norm"] if li + 1 < s.layers else self.w.final_norm
                o = self.be.single_raw(li, "o", self.attn, self.o_out)
                ck(lib.se12_step_rmsnorm(nat.ptr(o), dt(o), o.shape[1], nat.ptr(lw["post_attn_norm"]), nat.ptr(self.x),
                                         nat.ptr(lw["pre_ffw_norm"]), nat.ptr(self.h), B, s.hidden, s.eps, 0.0, 1, st))
                (g, go, gs), (u, uo, _) = self.be.grouped_raw(li, ("gate", "up"), self.h, self.gu)
                ck(lib.se12_step_gelu_mul(at(g, go), at(u, uo), dt(g), gs, nat.ptr(self.m), B, s.intermediate, st))
                dn = self.be.single_raw(li, "down", self.m, self.down_out)
                ck(lib.se12_step_rmsnorm(nat.ptr(dn), dt(dn), dn.shape[1], nat.ptr(lw["post_ffw_norm"]),
                                         nat.ptr(self.x), nat.ptr(nxt), nat.ptr(self.h), B, s.hidden, s.eps, 0.0, 1, st))
        lg = self.be.logits_raw(self.h, self.logits_out)
        ck(lib.se12_step_logits_argmax_advance(nat.ptr(lg), dt(lg), lg.shape[1], B, s.vocab, s.final_softcap,
                                               nat.ptr(self.last_logits), nat.ptr(self.ids), nat.ptr(self.tokens),
                                               self.max_len, nat.ptr(self.step_index), nat.ptr(self.pos),
                                               nat.ptr(self.logits_ws), self.logits_ws.numel(), st))

    def _attention(self, li: int, q_ptr: int, k_ptr: int, v_ptr: int, dtype: int, q_stride: int, kv_stride: int) -> None:
        s = self.s
        nat.step_check(nat.lib().se12_step_attention(
            q_ptr, k_ptr, v_ptr, dtype, q_stride, kv_stride, nat.ptr(self.kt[li]), nat.ptr(self.v[li]),
            nat.ptr(self.inv_freq), nat.ptr(self.pos), nat.ptr(self.attn), self.batch, s.heads, s.kv_heads, s.head_dim,
            self.max_len, self.scaling, s.attn_softcap, 0 if li % 2 else s.sliding_window, nat.ptr(self.attn_ws),
            self.attn_ws.numel(), nat.stream_ptr()))

    def _layers_fused_tails(self) -> None:
        """The layers with the step folded into the library products: every
        norm but the last in the head of the product that reads it
        (se12_gemv_prenorm: q/k/v, gate/up), the MLP gate in the gate/up
        tail, the final norm in the last down_proj's tail. 6 launches per
        layer: q/k/v, attention (2), o, gate/up, down."""
        from .hip import multiply_grouped, multiply_prenorm

        s = self.s
        ra, rb = self.x, self.x2     # the residual, and the buffer its update goes to
        for li, lw in enumerate(self.w.layers):
            ks = self.be.layers[li]
            qkv = [ks["q"], ks["k"], ks["v"]]
            if li == 0:
                multiply_grouped(qkv, self.h, outs=self.qkv)
            else:
                multiply_prenorm(qkv, self.down_out, self.w.layers[li - 1]["post_ffw_norm"], lw["input_norm"], ra, rb,
                                 self.h, s.eps, ys=self.qkv, y_prev_ss=self.down_ss)
                ra, rb = rb, ra
            q, k, v = self.qkv
            self._attention(li, q.data_ptr(), k.data_ptr(), v.data_ptr(), nat.STEP_F32, q.shape[1], k.shape[1])
            ks["o"].multiply_rowss(self.attn, self.o_ss, y=self.o_out)
            multiply_prenorm([ks["gate"], ks["up"]], self.o_out, lw["post_attn_norm"], lw["pre_ffw_norm"], ra, rb, self.h,
                             s.eps, ys=self.gu, gelu_out=self.m, y_prev_ss=self.o_ss)
            ra, rb = rb, ra
            if li + 1 < s.layers:
                ks["down"].multiply_rowss(self.m, self.down_ss, y=self.down_out)
            else:
                ks["down"].multiply_rmsnorm(self.m, lw["post_ffw_norm"], self.w.final_norm, ra, self.h, s.eps,
                                            y=self.down_out)
        self.residual = ra

    def step(self) -> None:
        """One decode step, eagerly (fused step kernels, or framework ops)."""
        if self.fused_step:
            self._step_fused()
        else:
            self._step()

    @torch.no_grad()
    def capture(self) -> None:
        """Captures one decode step; the KV cache and counters are restored
        afterwards (capture and its warm-up run the step twice)."""
        saved = (self.ids.clone(), self.pos.clone(), self.step_index.clone(), self.tokens.clone(),
                 [t.clone() for t in self.kt], [t.clone() for t in self.v])
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.step()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        torch.cuda.synchronize()
        self.ids.copy_(saved[0]); self.pos.copy_(saved[1]); self.step_index.copy_(saved[2]); self.tokens.copy_(saved[3])
        for t, c in zip(self.kt, saved[4]):
            t.copy_(c)
        for t, c in zip(self.v, saved[5]):
            t.copy_(c)
        self.graph = g

    @torch.no_grad()
    def decode(self, steps: int, graph: bool = True) -> None:
        """`steps` greedy steps after prefill (tokens land in self.tokens)."""
        if int(self.pos.item()) + steps > self.max_len:
            raise ValueError("the KV cache is too short for that many steps")
        for _ in range(steps):
            if graph:
                self.graph.replay()
            else:
                self.step()
