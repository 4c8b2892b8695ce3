"""The graph-captured Gemma-2 decode stack (se12_amd.gemma2) on a small shape:
- the SE12 backend and the order-matched raw-BF16 twin give bit-identical
  logits and the same greedy tokens over graph-replayed decode steps, with
  the step kernels and with framework ops around the products;
- graph replays give exactly what eager steps give;
- a step through the step kernels agrees with the framework-op step from the
  same state (logits and the KV-cache slot within BF16 rounding, for every
  backend);
- prefill and a decode step agree with transformers' Gemma2ForCausalLM on the
  same weights (attention with a contiguous key operand) within BF16
  rounding."""

from __future__ import annotations

import pytest
import torch

from se12_amd.gemma2 import PROJECTIONS, Gemma2Decoder, Gemma2Shape, Gemma2Weights

pytestmark = pytest.mark.gpu

TINY = Gemma2Shape(layers=2, hidden=256, intermediate=512, heads=4, kv_heads=2, head_dim=64, vocab=512)


def _encoded(w):
    from se12_amd.hip import encode_on_device

    enc = {(li, n): encode_on_device(lw[n]) for li, lw in enumerate(w.layers) for n in PROJECTIONS}
    enc["embed"] = encode_on_device(w.embed)
    return enc


def _prompt(gpu, batch, length, seed=3):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    return torch.randint(0, TINY.vocab, (batch, length), generator=g, device=gpu)


@pytest.mark.parametrize("batch,fused", [(1, True), (3, True), (3, False)])
def test_se12_and_raw_twin_decode_bit_identically(gpu, batch, fused):
    w = Gemma2Weights.random(TINY, gpu, seed=1)
    enc = _encoded(w)
    prompt = _prompt(gpu, batch, 12)
    out = {}
    for backend in ("se12", "raw"):
        d = Gemma2Decoder(w, backend, batch, max_len=32, encoded=enc, fused_step=fused)
        d.prefill(prompt)
        d.capture()
        d.decode(10)
        torch.cuda.synchronize()
        out[backend] = (d.tokens[:, :11].clone(), d.last_logits.clone())
    assert torch.equal(out["se12"][0], out["raw"][0])
    assert torch.equal(out["se12"][1], out["raw"][1])


@pytest.mark.parametrize("backend,fused", [("se12", True), ("se12", False), ("bf16", True)])
def test_graph_replays_equal_eager_steps(gpu, backend, fused):
    w = Gemma2Weights.random(TINY, gpu, seed=2)
    enc = _encoded(w)
    prompt = _prompt(gpu, 2, 9)
    a = Gemma2Decoder(w, backend, 2, max_len=24, encoded=enc, fused_step=fused)
    a.prefill(prompt)
    a.capture()
    a.decode(6)
    b = Gemma2Decoder(w, backend, 2, max_len=24, encoded=enc, fused_step=fused)
    b.prefill(prompt)
    b.decode(6, graph=False)
    torch.cuda.synchronize()
    assert torch.equal(a.tokens, b.tokens) and torch.equal(a.last_logits, b.last_logits)
    assert int(a.pos.item()) == 9 + 6


def _close(a: torch.Tensor, b: torch.Tensor, rel: float = 0.02) -> bool:
    a, b = a.float(), b.float()
    return (a - b).abs().max().item() <= rel * max(b.abs().max().item(), 1e-3)


@pytest.mark.parametrize("backend", ["se12", "raw", "bf16"])
def test_step_kernels_agree_with_the_framework_step(gpu, backend):
    """From one prefilled state, one step through the step kernels and one
    through framework ops: the same KV-cache slot and logits up to BF16
    rounding differences (FP32 sums in another order), propagated through
    the layers."""
    w = Gemma2Weights.random(TINY, gpu, seed=6)
    for lw in w.layers:
        for nm in ("input_norm", "post_attn_norm", "pre_ffw_norm", "post_ffw_norm"):
            lw[nm].normal_(0.0, 0.1)
    enc = _encoded(w) if backend == "se12" else None
    prompt = _prompt(gpu, 2, 11, seed=8)
    dec = {}
    for fused in (True, False):
        d = Gemma2Decoder(w, backend, 2, max_len=16, encoded=enc, fused_step=fused)
        d.prefill(prompt)
        d.decode(1, graph=False)
        torch.cuda.synchronize()
        dec[fused] = d
    a, b = dec[True], dec[False]
    assert int(a.pos.item()) == int(b.pos.item()) == 12 and int(a.step_index.item()) == 2
    for li in range(TINY.layers):
        # the prompt's slots are untouched; slot 11 is the new token's
        assert torch.equal(a.kt[li][..., :11], b.kt[li][..., :11]) and torch.equal(a.v[li][:, :, :11], b.v[li][:, :, :11])
        assert torch.equal(a.kt[li][..., 12:], b.kt[li][..., 12:])
        assert _close(a.kt[li][..., 11], b.kt[li][..., 11]) and _close(a.v[li][:, :, 11], b.v[li][:, :, 11])
    assert _close(a.last_logits, b.last_logits)
    # the argmax is the first maximum of each decoder's own logits
    for d in (a, b):
        mx = d.last_logits.float().max(dim=1, keepdim=True).values
        assert torch.equal(d.tokens[:, 1], (d.last_logits.float() == mx).float().argmax(dim=1))


def test_agrees_with_transformers_gemma2(gpu):
    from transformers import AutoModelForCausalLM, Gemma2Config

    from se12_amd import runtime

    w = Gemma2Weights.random(TINY, gpu, seed=4)
    for lw in w.layers:       # non-zero norm weights exercise the (1 + w) scaling
        for nm in ("input_norm", "post_attn_norm", "pre_ffw_norm", "post_ffw_norm"):
            lw[nm].normal_(0.0, 0.1)
    cfg = Gemma2Config(vocab_size=TINY.vocab, hidden_size=TINY.hidden, intermediate_size=TINY.intermediate,
                       num_hidden_layers=TINY.layers, num_attention_heads=TINY.heads,
                       num_key_value_heads=TINY.kv_heads, head_dim=TINY.head_dim,
                       attn_implementation=runtime.register_attention())
    hf = AutoModelForCausalLM.from_config(cfg, dtype=torch.bfloat16).to(gpu).eval()
    with torch.no_grad():
        for li, layer in enumerate(hf.model.layers):
            lw = w.layers[li]
            for mod, name in ((layer.self_attn.q_proj, "q"), (layer.self_attn.k_proj, "k"),
                              (layer.self_attn.v_proj, "v"), (layer.self_attn.o_proj, "o"),
                              (layer.mlp.gate_proj, "gate"), (layer.mlp.up_proj, "up"),
                              (layer.mlp.down_proj, "down")):
                mod.weight.copy_(lw[name])
            layer.input_layernorm.weight.copy_(lw["input_norm"])
            layer.post_attention_layernorm.weight.copy_(lw["post_attn_norm"])
            layer.pre_feedforward_layernorm.weight.copy_(lw["pre_ffw_norm"])
            layer.post_feedforward_layernorm.weight.copy_(lw["post_ffw_norm"])
        hf.model.embed_tokens.weight.copy_(w.embed)
        hf.model.norm.weight.copy_(w.final_norm)
    prompt = _prompt(gpu, 1, 14, seed=5)
    d = Gemma2Decoder(w, "bf16", 1, max_len=20, encoded=None)
    first = d.prefill(prompt)
    with torch.no_grad():
        ref = hf(prompt).logits[:, -1].float()
    lean = d.last_logits.float()
    scale = ref.abs().max().item()
    assert (lean - ref).abs().max().item() <= 0.02 * max(scale, 1.0)
    d.decode(1, graph=False)
    with torch.no_grad():
        ref2 = hf(torch.cat([prompt, first.view(1, 1)], dim=1)).logits[:, -1].float()
    assert (d.last_logits.float() - ref2).abs().max().item() <= 0.02 * max(ref2.abs().max().item(), 1.0)


def test_fused_tails_agree_with_separate_step_kernels(gpu):
    """The products with the residual norms in their heads and tails and the
    MLP gate in their tails against the same step with those as separate
    kernels: layer 0's K/V slot (before any of them) bit-identical, the rest
    within BF16 rounding."""
    w = Gemma2Weights.random(TINY, gpu, seed=9)
    enc = _encoded(w)
    prompt = _prompt(gpu, 1, 10, seed=5)
    ds = []
    for tails in (True, False):
        d = Gemma2Decoder(w, "se12", 1, max_len=24, encoded=enc, fused_tails=tails)
        assert d.fused_tails == tails
        d.prefill(prompt)
        d.decode(1, graph=False)
        torch.cuda.synchronize()
        ds.append(d)
    a, b = ds
    assert torch.equal(a.kt[0], b.kt[0]) and torch.equal(a.v[0], b.v[0])
    assert _close(a.kt[1][..., 10], b.kt[1][..., 10]) and _close(a.v[1][:, :, 10], b.v[1][:, :, 10])
    assert _close(a.residual, b.residual) and _close(a.last_logits, b.last_logits)
