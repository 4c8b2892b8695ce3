"""The runtime on the GPU with the library's kernels, on a small random-init
Hugging Face Gemma-2 (BF16; eager attention with a contiguous key operand):
- exact mode gives the original model's logits bit for bit (AC-016);
- fused mode with order="matched" against the reference runtime (original
  weights, raw-BF16 twin) gives identical logits at every greedy step and the
  same tokens (AC-033), and stays within rounding of the original model;
- auto mode follows this GPU's verdict file (AC-025);
- weights in HBM are at most 80% of the original's (AC-015)."""

from __future__ import annotations

import pytest
import torch

from se12_amd import runtime

pytestmark = pytest.mark.gpu


def _tiny_gemma(device, seed=0, layers=2):
    from transformers import AutoModelForCausalLM, Gemma2Config

    # attention with a contiguous key operand (see runtime.register_attention)
    cfg = Gemma2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                       attn_implementation=runtime.register_attention())
    torch.manual_seed(seed)
    model = AutoModelForCausalLM.from_config(cfg, dtype=torch.bfloat16)
    with torch.no_grad():
        for n, p in model.named_parameters():
            p.normal_(0.0, 0.02 if p.dim() == 2 else 0.1)
    return model.to(device).eval(), cfg


def _generate(model, ids, n):
    out = model.generate(ids, max_new_tokens=n, do_sample=False, output_logits=True, return_dict_in_generate=True)
    return out.sequences, torch.stack(out.logits)


def test_exact_mode_reproduces_the_original(gpu, tmp_path):
    model, cfg = _tiny_gemma(gpu)
    runtime.pack_pretrained(model, tmp_path / "packed")
    packed = runtime.load_packed(tmp_path / "packed", mode="exact", device=gpu, log=None, attn_implementation=runtime.register_attention())
    ids = torch.randint(0, cfg.vocab_size, (1, 24), device=gpu, generator=torch.Generator(device=gpu).manual_seed(1))
    with torch.no_grad():
        assert torch.equal(model(ids).logits, packed(ids).logits)
        sa, la = _generate(model, ids, 8)
        sb, lb = _generate(packed, ids, 8)
    assert torch.equal(sa, sb) and torch.equal(la, lb)
    wb = runtime.weight_bytes(packed)
    assert wb["total"] <= 0.8 * wb["original_total"]


@pytest.mark.parametrize("batch", [1, 6])
def test_matched_fused_mode_equals_the_reference_runtime(gpu, tmp_path, batch):
    model, cfg = _tiny_gemma(gpu, seed=5)
    runtime.pack_pretrained(model, tmp_path / "packed")
    model.save_pretrained(tmp_path / "orig")
    fused = runtime.load_packed(tmp_path / "packed", mode="fused", order="matched", device=gpu, log=None,
                                 attn_implementation=runtime.register_attention())
    ref = runtime.load_reference(tmp_path / "orig", device=gpu, order="matched", attn_implementation=runtime.register_attention())
    ids = torch.randint(0, cfg.vocab_size, (batch, 16), device=gpu, generator=torch.Generator(device=gpu).manual_seed(2))
    with torch.no_grad():
        sf, lf = _generate(fused, ids, 12)
        sr, lr = _generate(ref, ids, 12)
        so, lo = _generate(model, ids, 12)
    assert torch.equal(lf, lr) and torch.equal(sf, sr)
    # against the stock path only rounding differs: logits close at step 0
    assert (lf[0].float() - lo[0].float()).abs().max().item() < 0.05


def test_auto_mode_follows_the_verdict_file(gpu, tmp_path):
    model, cfg = _tiny_gemma(gpu, seed=7, layers=1)
    runtime.pack_pretrained(model, tmp_path / "packed")
    slug = runtime.current_gpu_slug(gpu)
    none = runtime.load_packed(tmp_path / "packed", mode="auto", device=gpu, verdict_dir=tmp_path / "v", log=None,
                                attn_implementation=runtime.register_attention())
    assert not none.lm_head.uses_fused(1, False)
    runtime.write_verdict(runtime.verdict_payload(slug, "gfx950", {1: [((512, 256), 0.6)], 4: [((512, 256), 1.1)],
                                                                  16: [((512, 256), 0.7)]}), tmp_path / "v")
    auto = runtime.load_packed(tmp_path / "packed", mode="auto", device=gpu, verdict_dir=tmp_path / "v", log=None,
                                attn_implementation=runtime.register_attention())
    lin = auto.lm_head
    assert [lin.uses_fused(b, False) for b in (1, 2, 4, 5, 16, 17)] == [True, False, False, True, True, False]
    assert not lin.uses_fused(1, True)     # prefill is always exact
    ids = torch.randint(0, cfg.vocab_size, (1, 8), device=gpu)
    with torch.no_grad():
        s_auto, _ = _generate(auto, ids, 4)
        s_none, _ = _generate(none, ids, 4)
    assert s_auto.shape == s_none.shape


def test_compressed_embedding_decodes_only_the_rows_asked_for(gpu, tmp_path):
    model, cfg = _tiny_gemma(gpu, seed=9, layers=1)
    runtime.pack_pretrained(model, tmp_path / "packed")
    packed = runtime.load_packed(tmp_path / "packed", mode="exact", device=gpu, log=None, attn_implementation=runtime.register_attention())
    ids = torch.tensor([[0, 511, 3, 3, 256]], device=gpu)
    with torch.no_grad():
        assert torch.equal(packed.model.embed_tokens(ids), model.model.embed_tokens(ids))


def test_tuned_configurations_are_consumed_and_stay_order_matched(gpu, tmp_path):
    """The tuner's file for this GPU (real evaluators) feeds both runtimes:
    fused layers launch with the order-matched entries, the reference runtime
    too, and the logits still agree bit for bit (AC-024 consumed, AC-033)."""
    from se12_amd import tune

    model, cfg = _tiny_gemma(gpu, seed=11)
    runtime.pack_pretrained(model, tmp_path / "packed")
    model.save_pretrained(tmp_path / "orig")
    shapes = {(256, 256), (128, 256), (512, 256), (256, 512)}
    reqs = [tune.tune_request(r, c, b) for r, c in sorted(shapes) for b in (1, 2)]
    slug = runtime.current_gpu_slug(gpu)
    tf = tune.tune_launch(slug, reqs, tune.gpu_evaluators(gpu, samples=3),
                          tune.FilesystemTuningCache(tmp_path / "t", slug))
    assert len(tf.entries.items) == len(reqs)
    attn = runtime.register_attention()
    fused = runtime.load_packed(tmp_path / "packed", mode="fused", order="matched", device=gpu, log=None,
                                attn_implementation=attn, tuning_dir=tmp_path / "t")
    ref = runtime.load_reference(tmp_path / "orig", device=gpu, order="matched", attn_implementation=attn,
                                 tuning_dir=tmp_path / "t")
    q = fused.model.layers[0].self_attn.q_proj
    assert q.launch_lookup(256, 256, 1) == tune.tuning_lookup(tf, "order_matched")(256, 256, 1)
    ids = torch.randint(0, cfg.vocab_size, (2, 10), device=gpu, generator=torch.Generator(device=gpu).manual_seed(4))
    with torch.no_grad():
        sf, lf = _generate(fused, ids, 6)
        sr, lr = _generate(ref, ids, 6)
    assert torch.equal(lf, lr) and torch.equal(sf, sr)
