"""The runtime's host logic on the CPU: the auto-mode policy and verdict files
(AC-025), and `load_packed`'s module surgery on a small random-init Hugging
Face Gemma-2 - every eligible Linear and the embedding replaced, the tied LM
head sharing the embedding's streams, pass-through tensors and rotary
buffers restored - with exact mode reproducing the original model's logits
bit for bit (AC-016). The GPU kernels are stood in for by an object that
decodes through the oracle (test infrastructure only)."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import se12_codec as o
from se12_amd import runtime
from se12_amd.format import packed_byte_size
from se12_amd.packed import PackedModel, is_eligible


def test_policy_follows_the_smallest_measured_batch_at_or_above():
    p = runtime.FusedPolicy(frozenset({1, 16}))
    assert [p.fused_for(b) for b in (1, 2, 4, 5, 16, 17, 32)] == [True, False, False, True, True, False, False]
    assert not any(runtime.FusedPolicy().fused_for(b) for b in (1, 4, 16))


def test_verdict_files_round_trip_and_other_gpus_are_ignored(tmp_path):
    ratios = {1: [((2304, 9216), 0.7), ((9216, 2304), 0.8)], 4: [((2304, 9216), 0.9), ((9216, 2304), 0.97)],
              16: [((2304, 9216), 0.5)]}
    payload = runtime.verdict_payload("amd-instinct-mi355x-gfx950", "gfx950", ratios)
    assert payload["verdict"] == "GO" and payload["per_batch"]["4"]["verdict"] == "NO-GO"
    assert payload["per_shape"] == [{"ratio": 0.7, "verdict": "GO"}, {"ratio": 0.8, "verdict": "GO"}]
    path = runtime.write_verdict(payload, tmp_path)
    assert path.name == "verdict-amd-instinct-mi355x-gfx950.json"
    p = runtime.load_policy("amd-instinct-mi355x-gfx950", tmp_path)
    assert p.go_batches == frozenset({1, 16}) and p.source == str(path)
    assert runtime.load_policy("some-other-gpu-gfx942", tmp_path).go_batches == frozenset()
    # a reference-style file (batch 1 only)
    (tmp_path / "verdict-x-gfx950.json").write_text(json.dumps({"gpu_slug": "x-gfx950", "verdict": "GO", "per_shape": []}))
    assert runtime.load_policy("x-gfx950", tmp_path).go_batches == frozenset({1})
    assert runtime.aggregate_verdict([]) == "INCONCLUSIVE"
    assert runtime.aggregate_verdict(["GO", "INCONCLUSIVE"]) == "INCONCLUSIVE"


class _OracleKernel:
    """Stands in for the bound GPU kernel: decodes through the oracle."""

    def __init__(self, name, tensor, device, max_batch):
        s = tensor.streams
        shape = tensor.metadata.geometry.shape
        self.enc = {"sm": s.primary.sm.value, "ec": s.primary.ec.value, "esc": s.escape_handling.esc.value,
                    "fallback_bitmap": s.escape_handling.fallback.bitmap.value,
                    "fallback_raw": s.escape_handling.fallback.raw.value,
                    "codebook": np.array(tensor.metadata.codebook.exponents, dtype=np.uint8),
                    "shape": (shape.rows, shape.cols)}
        self.rows, self.cols, self.device = shape.rows, shape.cols, device
        self.w = torch.from_numpy(o.decode(self.enc).astype(np.int16)).view(torch.bfloat16)
        fb = int(np.unpackbits(self.enc["fallback_bitmap"]).sum())
        self.tensor = type("T", (), {"rows": self.rows, "cols": self.cols,
                                     "byte_size": lambda _s: packed_byte_size(self.rows, self.cols, fb)})()

    def decode_into(self, out):
        out.copy_(self.w)
        return out

    def decode_rows_into(self, idx, out):
        out.copy_(self.w[idx])
        return out

    def multiply(self, x, launch=None):
        return x.float() @ self.w.float().t()


def _tiny_gemma(seed=0):
    from transformers import AutoModelForCausalLM, Gemma2Config

    cfg = Gemma2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=64, attn_implementation="eager")
    torch.manual_seed(seed)
    model = AutoModelForCausalLM.from_config(cfg, dtype=torch.bfloat16)
    with torch.no_grad():
        for n, p in model.named_parameters():
            if p.dim() == 2:
                p.normal_(0.0, 0.02)
            else:
                p.normal_(0.0, 0.1)
    return model.eval(), cfg


def _pack_with_oracle(model) -> PackedModel:
    tied = runtime._tied_names(model)
    se12, passthrough = {}, {}
    for name, t in model.state_dict().items():
        if name in tied:
            continue
        if is_eligible(t):
            bits = t.contiguous().view(torch.int16).numpy()
            enc = o.encode(bits.reshape(-1), *t.shape)
            from se12_amd.format import make_se12_tensor

            se12[name] = make_se12_tensor(enc["sm"], enc["ec"], enc["esc"], enc["fallback_bitmap"],
                                          enc["fallback_raw"], enc["codebook"], *t.shape)
        else:
            passthrough[name] = t.clone()
    return PackedModel(se12=se12, passthrough=passthrough, files=())


def test_load_packed_replaces_layers_and_exact_mode_matches_the_original():
    model, cfg = _tiny_gemma()
    pm = _pack_with_oracle(model)
    assert "lm_head.weight" not in pm.se12 and "model.embed_tokens.weight" in pm.se12
    packed = runtime.load_packed(pm, mode="exact", device="cpu", config=cfg, policy=runtime.FusedPolicy(),
                                 kernel_factory=_OracleKernel, log=None)
    lin = [n for n, m in packed.named_modules() if isinstance(m, runtime.CompressedLinear)]
    assert len(lin) == 2 * 7 + 1 and "lm_head" in lin
    assert isinstance(packed.model.embed_tokens, runtime.CompressedEmbedding)
    assert packed.lm_head.kernel is packed.model.embed_tokens.kernel   # tied: one set of streams
    assert not any(isinstance(m, torch.nn.Linear) for m in packed.modules())
    assert torch.equal(packed.model.rotary_emb.inv_freq, model.model.rotary_emb.inv_freq)
    wb = runtime.weight_bytes(packed)
    assert wb["total"] <= 0.8 * wb["original_total"]
    ids = torch.randint(0, cfg.vocab_size, (1, 12), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        a = model(ids).logits
        b = packed(ids).logits
    assert torch.equal(a, b)
    with torch.no_grad():
        ga = model.generate(ids, max_new_tokens=6, do_sample=False)
        gb = packed.generate(ids, max_new_tokens=6, do_sample=False)
    assert torch.equal(ga, gb)


def test_fused_mode_routes_decode_steps_to_the_kernel_and_prefill_to_exact():
    model, cfg = _tiny_gemma(seed=3)
    pm = _pack_with_oracle(model)
    calls = []

    class Counting(_OracleKernel):
        def multiply(self, x, launch=None):
            calls.append(tuple(x.shape))
            return super().multiply(x, launch)

    packed = runtime.load_packed(pm, mode="fused", device="cpu", config=cfg, policy=runtime.FusedPolicy(),
                                 kernel_factory=Counting, log=None)
    ids = torch.randint(0, cfg.vocab_size, (2, 5), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        packed(ids)
    assert calls == []                       # prefill: exact
    with torch.no_grad():
        packed.generate(ids, max_new_tokens=3, do_sample=False)
    assert calls and all(c[0] == 2 for c in calls)   # decode steps at batch 2
    with pytest.raises(ValueError):
        runtime.load_packed(pm, mode="fast", device="cpu", config=cfg, kernel_factory=Counting, log=None)
