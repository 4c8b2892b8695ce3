"""Per-GPU launch tuning and its cache file, consumed at run time.

The reference's tuner (lws/application/gpu/tune_launch.py:43-80) times every
candidate configuration of the raw and the fused kernel per (shape, batch),
keeps each kernel's fastest configuration that passes the accuracy check and
the best configuration shared by both (the order-matched one, AC-032), and
saves them through its TuningCache port (lws/application/ports/gpu/
tuning_cache.py:71-79), whose filesystem adapter writes `tune-<gpu-slug>.json`
(lws/adapters/filesystem/tuning_cache.py:31-160) - but nothing in the
reference loads that file back. Here:

- `tune_launch(gpu_slug, requests, evaluators, cache)` takes the reference's
  arguments: requests with `.weight_shape.output_rows`, `.weight_shape.k` and
  `.batch.value`; `evaluators(request)` returning an object with `.raw` and
  `.fused`, each a CandidateEvaluator (`.evaluate(configuration)` ->
  `.median_latency_microseconds`, `.passes_accuracy_check`); `cache` any
  TuningCache (`load()` / `save(tuning_file)`);
- `FilesystemTuningCache(directory, gpu_slug)` is that port on the file,
  with the reference's JSON layout and its rule for other GPUs' files (the
  first file recording this GPU's slug is used; otherwise one is named in a
  warning and None is returned);
- `tuning_lookup(tuning_file, kind)` turns a loaded file into the
  `launch_lookup` the runtime's layers call, and `load_packed` /
  `load_reference` read it for the current GPU.

The candidates are this kernel's (se12_amd.launch.candidate_configurations,
for BF16 and for FP32 activations: `tuning_candidates`);
the best and order-matched rules are the reference's, restated in
se12_amd.launch. The GPU evaluator times one launch per sample after a
read-only cache eviction (median over samples, HIP events) and passes a
configuration when its output is within 1e-3 x max(|y|, 1) of a float32
torch product of the decoded weights.

    python -m se12_amd.tune --shapes 2304x9216,9216x2304 --batches 1,4,16 --out reports
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import pathlib
import sys
import warnings
from typing import Any, Callable, Iterable, Sequence

import torch

from . import ports as P
from .launch import (
    BlockCount,
    LaunchConfiguration,
    ThreadsPerBlock,
    TimedCandidate,
    TimingAndAccuracy,
    best_configuration,
    candidate_configurations,
    order_matched_configuration,
)

KINDS = ("raw", "fused", "order_matched")
FILENAME_PREFIX = "tune-"
FILENAME_SUFFIX = ".json"


@dataclasses.dataclass(frozen=True)
class TuneRequest:
    """One (shape, batch) to tune (tune_launch.py:31-34)."""

    weight_shape: P.WeightShape
    batch: P.BatchSize


def tune_request(rows: int, cols: int, batch: int) -> TuneRequest:
    return TuneRequest(P.WeightShape(output_rows=int(rows), k=int(cols)), P.BatchSize(int(batch)))


@dataclasses.dataclass(frozen=True)
class EvaluatorPair:
    """The raw twin's and the fused kernel's evaluators (tune_launch.py:37-40)."""

    raw: Any
    fused: Any


def _kind_of(entry: Any, kind: str) -> LaunchConfiguration:
    c = entry.configurations
    if kind == "order_matched":
        return c.order_matched
    return getattr(c.independent, kind)


def entry_key(entry: Any) -> tuple[int, int, int]:
    """(rows, cols, batch) of a TunedEntry."""
    k = entry.key
    return int(k.weight_shape.output_rows), int(k.weight_shape.k), int(P.value_of(k.batch))


def tuning_lookup(tuning_file: Any, kind: str = "order_matched") -> Callable[[int, int, int], LaunchConfiguration | None]:
    """(rows, cols, batch) -> the tuned configuration of `kind` in a
    TuningFile, or None (the library default) for a shape it has no entry for."""
    if kind not in KINDS:
        raise ValueError(f"kind must be one of {KINDS}")
    table = {entry_key(e): _kind_of(e, kind) for e in tuning_file.entries.items}
    return lambda rows, cols, batch: table.get((rows, cols, batch))


def _cfg_to_json(c: Any) -> dict:
    return {"threads_per_block": int(c.threads_per_block.value), "blocks": int(c.blocks.value)}


def _cfg_from_json(d: dict) -> LaunchConfiguration:
    return LaunchConfiguration(ThreadsPerBlock(int(d["threads_per_block"])), BlockCount(int(d["blocks"])))


def to_json(tf: Any) -> dict:
    """The reference's file layout (tuning_cache.py:107-135)."""
    return {"gpu_slug": str(P.value_of(tf.gpu_slug)), "entries": [
        {"key": {"output_rows": r, "k": k, "batch": b},
         "configurations": {kind: _cfg_to_json(_kind_of(e, kind)) for kind in KINDS}}
        for e in tf.entries.items for (r, k, b) in [entry_key(e)]]}


def from_json(payload: dict) -> P.TuningFile:
    entries = []
    for raw in payload["entries"]:
        k, c = raw["key"], raw["configurations"]
        key = P.ShapeKey(P.WeightShape(int(k["output_rows"]), int(k["k"])), P.BatchSize(int(k["batch"])))
        conf = P.ConfigurationSet(
            independent=P.KernelConfigurations(raw=_cfg_from_json(c["raw"]), fused=_cfg_from_json(c["fused"])),
            order_matched=_cfg_from_json(c["order_matched"]))
        entries.append(P.TunedEntry(key=key, configurations=conf))
    return P.TuningFile(gpu_slug=P.GpuSlug(str(payload["gpu_slug"])), entries=P.TunedEntries(tuple(entries)))


def tuning_directory(directory=None) -> pathlib.Path:
    if directory is not None:
        return pathlib.Path(directory)
    return pathlib.Path(os.environ.get("LWS_TUNING_DIR", "reports"))


class FilesystemTuningCache:
    """TuningCache port (tuning_cache.py:71-79) on `<directory>/tune-<slug>.json`:
    `save` writes this GPU's file; `load` reads every `tune-*.json` there and
    returns the first (in name order) that records this GPU's slug, or None,
    warning about another GPU's file (lws/adapters/filesystem/
    tuning_cache.py:31-92). `gpu_slug` is a GpuSlug-like object or a str."""

    def __init__(self, directory: Any, gpu_slug: Any) -> None:
        self.directory = pathlib.Path(directory)
        self.gpu_slug = P.GpuSlug(str(P.value_of(gpu_slug)))

    def path(self) -> pathlib.Path:
        return self.directory / f"{FILENAME_PREFIX}{self.gpu_slug.value}{FILENAME_SUFFIX}"

    def load(self) -> P.TuningFile | None:
        candidates = sorted(self.directory.glob(f"{FILENAME_PREFIX}*{FILENAME_SUFFIX}")) if self.directory.exists() else []
        for path in candidates:
            payload = json.loads(path.read_text())
            if payload.get("gpu_slug") == self.gpu_slug.value:
                return from_json(payload)
        if candidates:
            found = json.loads(candidates[0].read_text()).get("gpu_slug")
            warnings.warn(f"ignoring tuning cache {candidates[0]}: it was recorded for GPU '{found}', "
                          f"current GPU is '{self.gpu_slug.value}'")
        return None

    def save(self, tuning_file: Any) -> None:
        self.directory.mkdir(parents=True, exist_ok=True)
        self.path().write_text(json.dumps(to_json(tuning_file), indent=2))


def _measure(evaluator: Any, cfg: LaunchConfiguration) -> TimingAndAccuracy:
    """One evaluation; a configuration the kernel refuses for the
    evaluator's activations (the library's validation raises) counts as
    failing, since evaluators need not catch it (the reference's does not,
    lws/adapters/cuda/candidate_evaluator.py:40-53)."""
    from ._native import Se12Error

    try:
        m = evaluator.evaluate(cfg) if hasattr(evaluator, "evaluate") else evaluator(cfg)
    except (ValueError, Se12Error):
        return TimingAndAccuracy(float("inf"), False)
    return TimingAndAccuracy(float(m.median_latency_microseconds), bool(m.passes_accuracy_check))


def tuning_candidates(rows: int, cols: int, batch: int) -> tuple[LaunchConfiguration, ...]:
    """The configurations timed per request: those of BF16 activations, then
    those only FP32 activations take (at 5+ rows BF16 runs an MFMA kernel and
    FP32 the dot2 kernel, whose configurations differ). A request does not
    say which the evaluators feed (the reference's tuner feeds FP32,
    lws/tune.py:80-83; this package's BF16), so both sets are offered and a
    kernel refuses the other's."""
    bf16 = candidate_configurations(rows, cols, batch=batch)
    seen = set(bf16)
    f32 = tuple(c for c in candidate_configurations(rows, cols, batch=batch, float32_activations=True) if c not in seen)
    return bf16 + f32


def tune_launch(gpu_slug: Any, requests: Sequence[Any], evaluators: Callable[[Any], Any], cache: Any) -> P.TuningFile:
    """Times every candidate of both kernels per request and keeps the
    fastest passing one of each and the best shared one; a request where
    nothing passes is left out. The file goes to `cache.save` and is
    returned (tune_launch.py:43-80)."""
    entries = []
    for req in requests:
        pair = evaluators(req)
        rows, cols = int(req.weight_shape.output_rows), int(req.weight_shape.k)
        batch = int(P.value_of(req.batch))
        cands = tuning_candidates(rows, cols, batch)
        raw_timed = tuple(TimedCandidate(c, _measure(pair.raw, c)) for c in cands)
        fused_timed = tuple(TimedCandidate(c, _measure(pair.fused, c)) for c in cands)
        best_raw, best_fused = best_configuration(raw_timed), best_configuration(fused_timed)
        matched = order_matched_configuration(raw_timed, fused_timed)
        if best_raw is None or best_fused is None or matched is None:
            continue
        key = P.ShapeKey(P.WeightShape(rows, cols), P.BatchSize(batch))
        conf = P.ConfigurationSet(independent=P.KernelConfigurations(raw=best_raw, fused=best_fused),
                                  order_matched=matched)
        entries.append(P.TunedEntry(key=key, configurations=conf))
    tf = P.TuningFile(gpu_slug=P.GpuSlug(str(P.value_of(gpu_slug))), entries=P.TunedEntries(tuple(entries)))
    cache.save(tf)
    return tf


class GpuEvaluator:
    """CandidateEvaluator (lws/application/ports/gpu/candidate_evaluator.py:
    15-17) over one bound kernel: `evaluate(configuration)` times its launch
    (median of `samples`, each after a cache eviction) and checks accuracy
    against a float32 product."""

    def __init__(self, kernel, x: torch.Tensor, reference: torch.Tensor, samples: int = 7, timer=None) -> None:
        from .hip import HipBenchmarkTimer

        self.kernel, self.x, self.ref = kernel, x, reference
        self.samples = samples
        self.timer = timer or HipBenchmarkTimer(x.device.index)
        self.scale = reference.abs().clamp_min(1.0)

    def evaluate(self, configuration: LaunchConfiguration) -> TimingAndAccuracy:
        y = torch.empty((self.x.shape[0], self.kernel.rows), dtype=torch.float32, device=self.x.device)
        try:
            self.kernel.multiply(self.x, launch=configuration, out=y)
            torch.cuda.synchronize(self.x.device)
        except Exception:
            return TimingAndAccuracy(float("inf"), False)
        ok = bool(((y - self.ref).abs() / self.scale).max().item() <= 1e-3)
        st = self.timer.time_stats(lambda: self.kernel.multiply(self.x, launch=configuration, out=y), warmup=2,
                                   timed=self.samples)
        return TimingAndAccuracy(st.median_us, ok)

    __call__ = evaluate


def gpu_evaluators(device, seed: int = 0, samples: int = 7):
    """request -> EvaluatorPair over random BF16 N(0, 0.02) weights of the
    requested shape (encoded on the GPU) and N(0, 1) activations."""
    from .hip import HipBenchmarkTimer, RawBf16MatVecKernel, Se12MatVecKernel, encode_on_device

    timer = HipBenchmarkTimer(torch.device(device).index)
    cache: dict = {}

    def make(req) -> EvaluatorPair:
        rows, cols = int(req.weight_shape.output_rows), int(req.weight_shape.k)
        batch = int(P.value_of(req.batch))
        key = (rows, cols)
        if key not in cache:
            g = torch.Generator(device=device)
            g.manual_seed(seed + rows * 7 + cols)
            w = (torch.randn((rows, cols), generator=g, device=device) * 0.02).to(torch.bfloat16)
            cache[key] = (w, Se12MatVecKernel(encode_on_device(w)), RawBf16MatVecKernel(w))
        w, fused, raw = cache[key]
        g = torch.Generator(device=device)
        g.manual_seed(seed + 1 + batch)
        x = torch.randn((batch, cols), generator=g, device=device).to(torch.bfloat16)
        ref = x.float() @ w.float().t()
        return EvaluatorPair(raw=GpuEvaluator(raw, x, ref, samples, timer), fused=GpuEvaluator(fused, x, ref, samples, timer))

    return make


def main(argv: Iterable[str] | None = None) -> int:
    p = argparse.ArgumentParser(description="tune SE12 launch configurations for this GPU")
    p.add_argument("--shapes", default="2048x2304,1024x2304,2304x2048,9216x2304,2304x9216")
    p.add_argument("--batches", default="1,4,16")
    p.add_argument("--out", default=None, help="directory of tune-<gpu-slug>.json (default $LWS_TUNING_DIR or reports)")
    p.add_argument("--samples", type=int, default=7)
    args = p.parse_args(list(argv) if argv is not None else None)
    from .runtime import current_gpu_slug

    dev = torch.device("cuda", torch.cuda.current_device())
    reqs = [tune_request(int(s.split("x")[0]), int(s.split("x")[1]), int(b))
            for s in args.shapes.split(",") for b in args.batches.split(",")]
    slug = current_gpu_slug(dev)
    cache = FilesystemTuningCache(tuning_directory(args.out), slug)
    tf = tune_launch(slug, reqs, gpu_evaluators(dev, samples=args.samples), cache)
    print(f"tuning written for GPU '{slug}' ({len(tf.entries.items)} of {len(reqs)} (shape, batch) combinations) "
          f"in {cache.path()}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
