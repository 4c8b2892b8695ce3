"""Drop-in compressed layers and the packed-model loader.

The reference specifies this runtime but does not implement it
(.spec/features/model-integration/spec.md: `lws.runtime.load_packed(packed_dir,
mode=..., order="matched")` AC-015/016/025/033, `load_reference(model_dir)`;
tasks.md:16 `CompressedLinear.forward`). Here:

- `CompressedLinear` keeps only the SE12 streams of a weight in HBM. Its
  forward takes one of two paths: *fused* (the library's fused decode +
  product, FP32 accumulate, rounded to the activation dtype) or *exact*
  (decode the layer into a scratch buffer shared by the whole model, then the
  same `F.linear` the original layer runs - bit-identical to the original).
- `mode="exact"` always takes the exact path, `mode="fused"` the fused path
  for every decode step, `mode="auto"` the fused path for a batch size b only
  where this GPU's verdict file records GO at the smallest measured batch
  size >= b (1, 4 or 16), exact otherwise and for every b > 16 (AC-025).
  Prefill (more than one new token per sequence) is always exact.
- `CompressedEmbedding` decodes only the rows it looks up (the tiles of those
  rows); a tied LM head is a `CompressedLinear` over the same streams.
- `load_reference` is the order-matched reference runtime: original BF16
  weights, decode steps through the raw-BF16 twin kernel (AC-033). With
  `order="matched"` both runtimes launch with one configuration per
  (shape, batch) - the library default, or the tuner's order-matched entry -
  so their logits agree bit for bit.

Verdict files: `verdict-<gpu-slug>.json` in `verdict_dir`, `$LWS_VERDICT_DIR`
or `reports/`, with the reference's batch-1 fields (gpu_slug, verdict,
per_shape; lws/bench/micro.py:215-228) plus `per_batch` {"1"|"4"|"16":
{"verdict": ..., "per_shape": [...]}} - the reference records batch 1 only.
A verdict is GO when every shape's fused/baseline median ratio is at most
0.95 (lws/domain/benchmark/verdict.py:8,57-85).
"""

from __future__ import annotations

import dataclasses
import json
import os
import pathlib
from typing import Any, Callable

import torch
import torch.nn.functional as F
from torch import nn

from . import _native as nat
from .format import Se12DeviceTensor
from .launch import LaunchConfiguration
from .packed import PackedModel, is_eligible, read_packed, write_packed_file

VERDICT_BATCHES = (1, 4, 16)
GO_RATIO_THRESHOLD = 0.95
# a comparison is valid only where the baseline reaches this fraction of the
# measured copy bandwidth (lws/domain/benchmark/verdict.py:12,40-50)
PEAK_BANDWIDTH_FRACTION = 0.70
MODES = ("exact", "fused", "auto")


# ---------------------------------------------------------------------------
# verdicts and the auto-mode policy
# ---------------------------------------------------------------------------


@dataclasses.dataclass(frozen=True)
class FusedPolicy:
    """Which decode batch sizes take the fused path (AC-025)."""

    go_batches: frozenset = frozenset()
    source: str | None = None

    def fused_for(self, batch: int) -> bool:
        for measured in VERDICT_BATCHES:
            if batch <= measured:
                return measured in self.go_batches
        return False

    def describe(self) -> dict:
        return {"source": self.source,
                "fused_batches": {b: self.fused_for(b) for b in (1, 2, 4, 8, 16, 17)}}


def shape_verdict(ratio: float, baseline_fraction_of_peak: float | None = None) -> str:
    """GO when the fused median is at most 0.95 x the faster lossless
    baseline's, NO-GO otherwise; INCONCLUSIVE when that baseline reaches less
    than 70% of the measured copy bandwidth (verdict.py:40-62)."""
    if baseline_fraction_of_peak is not None and baseline_fraction_of_peak < PEAK_BANDWIDTH_FRACTION:
        return "INCONCLUSIVE"
    return "GO" if ratio <= GO_RATIO_THRESHOLD else "NO-GO"


def aggregate_verdict(verdicts) -> str:
    verdicts = list(verdicts)
    if not verdicts or any(v == "INCONCLUSIVE" for v in verdicts):
        return "INCONCLUSIVE"
    return "GO" if all(v == "GO" for v in verdicts) else "NO-GO"


def verdict_payload(gpu_slug: str, arch: str, ratios: dict[int, list[tuple]]) -> dict:
    """The verdict file for one GPU from fused/baseline median ratios per
    batch size: {batch: [(shape, ratio) or (shape, ratio, baseline fraction
    of the measured copy peak), ...]}."""
    per_batch = {}
    for b, items in sorted(ratios.items()):
        per_shape = []
        for item in items:
            shape, r = item[0], float(item[1])
            frac = float(item[2]) if len(item) > 2 and item[2] is not None else None
            entry = {"shape": list(shape), "ratio": r, "verdict": shape_verdict(r, frac)}
            if frac is not None:
                entry["baseline_fraction_of_peak"] = frac
            per_shape.append(entry)
        per_batch[str(b)] = {"verdict": aggregate_verdict(p["verdict"] for p in per_shape), "per_shape": per_shape}
    one = per_batch.get("1", {"verdict": "INCONCLUSIVE", "per_shape": []})
    # compute_capability: the reference's field name (micro.py:215-228),
    # holding the gfx architecture here
    return {"gpu_slug": gpu_slug, "arch": arch, "compute_capability": arch, "verdict": one["verdict"],
            "per_shape": [{"ratio": p["ratio"], "verdict": p["verdict"]} for p in one["per_shape"]],
            "per_batch": per_batch}


def verdict_directory(directory=None) -> pathlib.Path:
    if directory is not None:
        return pathlib.Path(directory)
    return pathlib.Path(os.environ.get("LWS_VERDICT_DIR", "reports"))


def write_verdict(payload: dict, directory=None) -> pathlib.Path:
    d = verdict_directory(directory)
    d.mkdir(parents=True, exist_ok=True)
    path = d / f"verdict-{payload['gpu_slug']}.json"
    path.write_text(json.dumps(payload, indent=1))
    return path


def load_policy(gpu_slug: str, directory=None) -> FusedPolicy:
    """The auto-mode policy from this GPU's verdict file; without one (e.g.
    only another GPU's), every layer stays exact (AC-025)."""
    path = verdict_directory(directory) / f"verdict-{gpu_slug}.json"
    if not path.exists():
        return FusedPolicy(frozenset(), None)
    payload = json.loads(path.read_text())
    if payload.get("gpu_slug") != gpu_slug:
        return FusedPolicy(frozenset(), None)
    go = set()
    per_batch = payload.get("per_batch")
    if per_batch:
        for b, entry in per_batch.items():
            if int(b) in VERDICT_BATCHES and entry.get("verdict") == "GO":
                go.add(int(b))
    elif payload.get("verdict") == "GO":  # a batch-1-only verdict
        go.add(1)
    return FusedPolicy(frozenset(go), str(path))


def current_gpu_slug(device=None) -> str:
    from .hip import HipGpuProbe

    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    return HipGpuProbe(dev.index if dev.index is not None else torch.cuda.current_device()).facts().slug


# ---------------------------------------------------------------------------
# layers
# ---------------------------------------------------------------------------


class DecodeScratch:
    """One BF16 buffer per device that every exact-path layer of a model
    decodes into (grown to the largest layer), so no full BF16 weight stays
    resident. Uses are ordered on the stream that issues them."""

    def __init__(self) -> None:
        self._buf: dict[torch.device, torch.Tensor] = {}

    def take(self, rows: int, cols: int, device: torch.device) -> torch.Tensor:
        n = rows * cols
        buf = self._buf.get(device)
        if buf is None or buf.numel() < n:
            buf = torch.empty(n, dtype=torch.bfloat16, device=device)
            self._buf[device] = buf
        return buf[:n].view(rows, cols)

    def bytes(self) -> int:
        return sum(b.numel() * 2 for b in self._buf.values())


LaunchLookup = Callable[[int, int, int], "LaunchConfiguration | None"]


def _split_batch(x: torch.Tensor, cols: int) -> tuple[torch.Tensor, int, bool]:
    """[..., K] -> ([M, K], M, prefill): a 3-D input with more than one token
    per sequence is a prefill."""
    prefill = x.dim() >= 3 and x.shape[-2] > 1
    x2 = x.reshape(-1, cols)
    return x2, x2.shape[0], prefill


class CompressedLinear(nn.Module):
    """nn.Linear replacement holding SE12 streams only (AC-015)."""

    def __init__(self, kernel, bias: torch.Tensor | None = None, mode: str = "auto",
                 policy: FusedPolicy | None = None, scratch: DecodeScratch | None = None,
                 launch_lookup: LaunchLookup | None = None) -> None:
        super().__init__()
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
        self.kernel = kernel
        self.in_features, self.out_features = kernel.cols, kernel.rows
        self.mode = mode
        self.policy = policy if policy is not None else FusedPolicy()
        self.scratch = scratch if scratch is not None else DecodeScratch()
        self.launch_lookup = launch_lookup
        self.bias = nn.Parameter(bias, requires_grad=False) if bias is not None else None

    @property
    def tensor(self) -> Se12DeviceTensor:
        return self.kernel.tensor

    def uses_fused(self, batch: int, prefill: bool) -> bool:
        if self.mode == "exact" or prefill or batch > nat.MAX_BATCH:
            return False
        return self.mode == "fused" or self.policy.fused_for(batch)

    def decoded_weight(self) -> torch.Tensor:
        """The BF16 weight, decoded into the shared scratch (valid until the
        next exact-path layer decodes)."""
        w = self.scratch.take(self.out_features, self.in_features, self.kernel.device)
        return self.kernel.decode_into(w)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x2, m, prefill = _split_batch(x, self.in_features)
        if self.uses_fused(m, prefill):
            launch = self.launch_lookup(self.out_features, self.in_features, m) if self.launch_lookup else None
            y = self.kernel.multiply(x2, launch=launch)
            if self.bias is not None:
                y = y + self.bias.float()
            y = y.to(x.dtype)
        else:
            y = F.linear(x2, self.decoded_weight().to(x.dtype), self.bias)
        return y.reshape(*x.shape[:-1], self.out_features)

    def stream_bytes(self) -> int:
        return self.tensor.byte_size()

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, mode={self.mode}, se12"


class CompressedEmbedding(nn.Module):
    """nn.Embedding replacement: looks rows up by decoding only their tiles.
    `scale` reproduces scaled embeddings (Gemma's: rows x sqrt(hidden), the
    product taken in BF16 as the original module does)."""

    def __init__(self, kernel, padding_idx: int | None = None, scale: float | None = None) -> None:
        super().__init__()
        self.kernel = kernel
        self.num_embeddings, self.embedding_dim = kernel.rows, kernel.cols
        self.padding_idx = padding_idx
        self.scale = scale

    @property
    def tensor(self) -> Se12DeviceTensor:
        return self.kernel.tensor

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        idx = ids.reshape(-1).to(device=self.kernel.device, dtype=torch.int64).contiguous()
        out = torch.empty((idx.numel(), self.embedding_dim), dtype=torch.bfloat16, device=self.kernel.device)
        self.kernel.decode_rows_into(idx, out)
        if self.scale is not None:
            out = out * torch.tensor(self.scale, dtype=torch.bfloat16, device=out.device)
        return out.view(*ids.shape, self.embedding_dim)

    def stream_bytes(self) -> int:
        return self.tensor.byte_size()

    def extra_repr(self) -> str:
        return f"{self.num_embeddings}, {self.embedding_dim}, se12"


class ReferenceLinear(nn.Module):
    """The reference runtime's layer (AC-033): the original BF16 weight, decode
    steps through the raw-BF16 twin kernel, prefill through `F.linear`."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None,
                 launch_lookup: LaunchLookup | None = None) -> None:
        super().__init__()
        from .hip import RawBf16MatVecKernel

        self.weight = nn.Parameter(weight.detach().contiguous(), requires_grad=False)
        self.bias = nn.Parameter(bias.detach(), requires_grad=False) if bias is not None else None
        self.out_features, self.in_features = self.weight.shape
        self.kernel = RawBf16MatVecKernel(self.weight.data)
        self.launch_lookup = launch_lookup

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x2, m, prefill = _split_batch(x, self.in_features)
        if prefill or m > nat.MAX_BATCH:
            y = F.linear(x2, self.weight.to(x.dtype), self.bias)
        else:
            launch = self.launch_lookup(self.out_features, self.in_features, m) if self.launch_lookup else None
            y = self.kernel.multiply(x2, launch=launch)
            if self.bias is not None:
                y = y + self.bias.float()
            y = y.to(x.dtype)
        return y.reshape(*x.shape[:-1], self.out_features)


# ---------------------------------------------------------------------------
# packing and loading Hugging Face models
# ---------------------------------------------------------------------------

CONTIGUOUS_EAGER = "se12_eager"


def _contiguous_eager_attention(module, query, key, value, attention_mask, dropout=0.0, scaling=None,
                                softcap=None, **kwargs):
    """transformers' eager attention (with Gemma-2's logit soft-capping),
    computed the same way except that the transposed key is made contiguous
    before the batched product: BF16 batched products whose right operand is
    a transposed view have faulted the GPU on MI355X."""
    if scaling is None:
        scaling = module.head_dim ** -0.5
    groups = query.shape[1] // key.shape[1]
    if groups > 1:
        b, h, s, d = key.shape
        key = key[:, :, None].expand(b, h, groups, s, d).reshape(b, h * groups, s, d)
        value = value[:, :, None].expand(b, h, groups, s, d).reshape(b, h * groups, s, d)
    weights = torch.matmul(query, key.transpose(2, 3).contiguous()) * scaling
    if softcap is not None:
        weights = torch.tanh(weights / softcap) * softcap
    if attention_mask is not None:
        weights = weights + attention_mask
    weights = F.softmax(weights, dim=-1, dtype=torch.float32).to(query.dtype)
    weights = F.dropout(weights, p=dropout, training=module.training)
    out = torch.matmul(weights, value.contiguous())
    return out.transpose(1, 2).contiguous(), weights


# Attention implementations refused on a HIP device: transformers' eager
# attention multiplies BF16 query [B, H, S, D] by key.transpose(2, 3), a view
# with strides (H*S*D, S*D, 1, D); BF16 batched products whose right operand
# is such a view have faulted MI355X GPUs (torch 2.10.0+rocm7.0 on ROCm 7.2).
_FAULTING_ATTENTION = ("eager",)


def resolve_attention(attn_implementation: str | None, device: torch.device) -> str | None:
    """The attention implementation a model is built with: on a HIP device
    the contiguous-key eager attention ("se12_eager") unless the caller names
    another one, and never transformers' own "eager"."""
    if device.type != "cuda":
        return attn_implementation
    if attn_implementation is None:
        attn_implementation = CONTIGUOUS_EAGER
    if attn_implementation in _FAULTING_ATTENTION:
        raise ValueError(f"attn_implementation={attn_implementation!r} runs a BF16 batched product on a transposed "
                         f"key view, which has faulted MI355X GPUs; use {CONTIGUOUS_EAGER!r} (the same computation "
                         "with a contiguous key) or leave it None")
    if attn_implementation == CONTIGUOUS_EAGER:
        register_attention()
    return attn_implementation


def register_attention() -> str:
    """Registers the attention above with transformers as "se12_eager"; pass
    that name as `attn_implementation` to the original and the packed model
    alike."""
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, AttentionMaskInterface

    AttentionInterface.register(CONTIGUOUS_EAGER, _contiguous_eager_attention)
    # the additive masks eager attention gets (without a mask function of its
    # own, an implementation is handed no mask at all)
    AttentionMaskInterface.register(CONTIGUOUS_EAGER, ALL_MASK_ATTENTION_FUNCTIONS["eager"])
    return CONTIGUOUS_EAGER


def _module_and_attr(model: nn.Module, dotted: str) -> tuple[nn.Module, str]:
    parent, _, attr = dotted.rpartition(".")
    return (model.get_submodule(parent) if parent else model), attr


def _tied_names(model: nn.Module) -> dict[str, str]:
    """Parameter names that are the same parameter as an earlier name (a tied
    LM head) -> that name. By identity, so it also holds on the meta device."""
    seen: dict[int, str] = {}
    tied = {}
    for name, p in model.named_parameters(remove_duplicate=False):
        key = id(p)
        if key in seen and seen[key] != name:
            tied[name] = seen[key]
        else:
            seen.setdefault(key, name)
    return tied


def pack_pretrained(model: nn.Module, out_dir, device=None, shard_name: str = "model.safetensors") -> pathlib.Path:
    """Packs a Hugging Face model: eligible weights SE12-encoded on the GPU,
    everything else passed through, tied copies stored once; writes the
    model's config.json beside the container."""
    out = pathlib.Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    tied = _tied_names(model)
    sd = {k: v for k, v in model.state_dict().items() if k not in tied}
    from .packed import pack_state_dict

    pack_state_dict(sd, out / shard_name, device=device)
    if hasattr(model, "config"):
        model.config.save_pretrained(str(out))
    return out


def _reinit_rotary(model: nn.Module, device: torch.device) -> None:
    """Recomputes rotary inverse frequencies (non-persistent buffers, not in
    any checkpoint) after a model was materialised from the meta device: a
    fresh module of the same class is built from its config and its buffers
    and attention scaling copied over."""
    for mod in model.modules():
        if hasattr(mod, "inv_freq") and hasattr(mod, "config"):
            with torch.device("cpu"):
                fresh = type(mod)(mod.config)
            for name, buf in fresh.named_buffers(recurse=False):
                setattr(mod, name, buf.to(device))
            if hasattr(fresh, "attention_scaling"):
                mod.attention_scaling = fresh.attention_scaling


def _default_kernel(name: str, tensor, device: torch.device, max_batch: int):
    from .hip import Se12MatVecKernel

    return Se12MatVecKernel(Se12DeviceTensor.from_host(tensor, device), max_batch=max_batch)


def load_packed(packed: Any, mode: str = "auto", order: str | None = None, device=None, config=None,
                policy: FusedPolicy | None = None, verdict_dir=None, launch_lookup: LaunchLookup | None = None,
                max_batch: int = nat.MAX_BATCH, log: Callable[[str], None] | None = print,
                kernel_factory: Callable[[str, Any, torch.device, int], Any] | None = None,
                attn_implementation: str | None = None, tuning_dir=None) -> nn.Module:
    """A Hugging Face causal LM whose eligible Linear and Embedding layers are
    SE12-backed (AC-015): `packed` is a packed directory/file or a
    `PackedModel`; `config` defaults to the directory's config.json.
    `order="matched"` launches every fused step with the configuration the
    reference runtime uses. Launch configurations come from `launch_lookup`,
    else this GPU's tuning file (`tune-<gpu-slug>.json` in `tuning_dir`,
    $LWS_TUNING_DIR or reports/: its order-matched entries with
    order="matched", its fused entries otherwise), else the library default."""
    from transformers import AutoConfig, AutoModelForCausalLM

    if mode not in MODES:
        raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
    if order not in (None, "matched"):
        raise ValueError(f"order must be None or 'matched', got {order!r}")
    pm = packed if isinstance(packed, PackedModel) else read_packed(packed)
    if config is None:
        if isinstance(packed, PackedModel):
            raise ValueError("a config is needed when loading from a PackedModel")
        config = AutoConfig.from_pretrained(str(packed))
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if policy is None:
        policy = load_policy(current_gpu_slug(dev), verdict_dir) if mode == "auto" else FusedPolicy()
    if launch_lookup is None and mode != "exact" and kernel_factory is None:
        launch_lookup = tuned_lookup(dev, "order_matched" if order == "matched" else "fused", tuning_dir)
    make_kernel = kernel_factory or _default_kernel
    attn_implementation = resolve_attention(attn_implementation, dev)
    extra = {"attn_implementation": attn_implementation} if attn_implementation else {}
    with torch.device("meta"):
        model = AutoModelForCausalLM.from_config(config, dtype=torch.bfloat16, **extra)
    scratch = DecodeScratch()
    kernels: dict[str, Any] = {}

    def kernel_for(name: str):
        if name not in kernels:
            kernels[name] = make_kernel(name, pm.se12[name], dev, max_batch)
        return kernels[name]

    tied = _tied_names(model)
    replaced = set()
    for name, mod in list(model.named_modules()):
        wname = f"{name}.weight"
        src = wname if wname in pm.se12 else tied.get(wname) if tied.get(wname) in pm.se12 else None
        if src is None:
            continue
        parent, attr = _module_and_attr(model, name)
        if isinstance(mod, nn.Linear):
            # a bias stays an ordinary parameter, filled from its pass-through
            # tensor after the model is materialised
            bias = torch.empty(mod.out_features, dtype=torch.bfloat16, device="meta") if mod.bias is not None else None
            new = CompressedLinear(kernel_for(src), bias, mode=mode, policy=policy, scratch=scratch,
                                   launch_lookup=launch_lookup)
        elif isinstance(mod, nn.Embedding):
            # a scaled embedding keeps its scale in a non-persistent buffer that
            # no checkpoint holds; Gemma models set it to sqrt(hidden_size)
            scale = float(config.hidden_size) ** 0.5 if hasattr(mod, "embed_scale") else None
            new = CompressedEmbedding(kernel_for(src), padding_idx=mod.padding_idx, scale=scale)
        else:
            raise ValueError(f"{wname} is SE12 but {name} is a {type(mod).__name__}")
        setattr(parent, attr, new)
        replaced.add(wname)
    model.to_empty(device=dev)
    for name, t in pm.passthrough.items():
        if name in replaced:
            continue
        parent, attr = _module_and_attr(model, name)
        target = getattr(parent, attr, None)
        if not isinstance(target, torch.Tensor):
            raise ValueError(f"pass-through tensor {name!r} has no counterpart in the model")
        if tuple(target.shape) != tuple(t.shape):
            raise ValueError(f"{name}: model expects {tuple(target.shape)}, file holds {tuple(t.shape)}")
        with torch.no_grad():
            target.copy_(t.to(device=dev, dtype=target.dtype))
    missing = [n for n, _ in model.named_parameters() if n not in pm.passthrough and n not in tied]
    if missing:
        raise ValueError(f"parameters with no packed tensor: {missing[:5]}")
    _reinit_rotary(model, dev)
    model.eval()
    model.se12_policy = policy
    model.se12_scratch = scratch
    if log is not None:
        n_lin = sum(isinstance(m, CompressedLinear) for m in model.modules())
        log(f"[se12] load_packed: {n_lin} CompressedLinear, mode={mode}, order={order}, "
            f"policy {policy.describe()}")
    return model


def tuned_lookup(device, kind: str, tuning_dir=None) -> LaunchLookup | None:
    """The launch lookup of this GPU's tuning file, or None without one."""
    from .tune import FilesystemTuningCache, tuning_directory, tuning_lookup

    tf = FilesystemTuningCache(tuning_directory(tuning_dir), current_gpu_slug(device)).load()
    return tuning_lookup(tf, kind) if tf is not None else None


def load_reference(model_dir, device=None, order: str | None = "matched",
                   launch_lookup: LaunchLookup | None = None, model: nn.Module | None = None,
                   attn_implementation: str | None = None, tuning_dir=None) -> nn.Module:
    """The reference runtime (AC-033): original BF16 weights, every eligible
    Linear through the raw-BF16 twin for decode steps, launched with the
    tuning file's order-matched (order="matched") or raw entries when this GPU
    has one."""
    from transformers import AutoModelForCausalLM

    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if launch_lookup is None:
        launch_lookup = tuned_lookup(dev, "order_matched" if order == "matched" else "raw", tuning_dir)
    attn_implementation = resolve_attention(attn_implementation, dev)
    if model is None:
        extra = {"attn_implementation": attn_implementation} if attn_implementation else {}
        model = AutoModelForCausalLM.from_pretrained(str(model_dir), dtype=torch.bfloat16, **extra)
    elif dev.type == "cuda" and getattr(model.config, "_attn_implementation", None) in _FAULTING_ATTENTION:
        raise ValueError(f"the model was built with attn_implementation={model.config._attn_implementation!r}, which "
                         f"faults MI355X GPUs; build it with {CONTIGUOUS_EAGER!r} (runtime.register_attention())")
    model = model.to(dev)
    for name, mod in list(model.named_modules()):
        if isinstance(mod, nn.Linear) and is_eligible(mod.weight):
            parent, attr = _module_and_attr(model, name)
            setattr(parent, attr, ReferenceLinear(mod.weight.data, mod.bias.data if mod.bias is not None else None,
                                                  launch_lookup=launch_lookup))
    model.eval()
    return model


def weight_bytes(model: nn.Module) -> dict:
    """Bytes of weights resident in HBM: SE12 streams (each bound tensor once)
    plus the remaining parameters, against the BF16 bytes they replace."""
    seen = set()
    se12 = bf16 = 0
    for m in model.modules():
        if isinstance(m, (CompressedLinear, CompressedEmbedding)):
            t = m.tensor
            if id(t) in seen:
                continue
            seen.add(id(t))
            se12 += t.byte_size()
            bf16 += 2 * t.rows * t.cols
    other = sum(p.numel() * p.element_size() for n, p in model.named_parameters())
    return {"se12_bytes": se12, "replaced_bf16_bytes": bf16, "other_parameter_bytes": other,
            "total": se12 + other, "original_total": bf16 + other}


def save_packed(model_se12: dict, passthrough: dict, path) -> pathlib.Path:
    """Writes already-encoded host tensors (see `packed.write_packed_file`)."""
    return write_packed_file(path, model_se12, passthrough)
