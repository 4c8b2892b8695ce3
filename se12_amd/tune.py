"""Per-GPU launch tuning and its cache file, consumed at run time.

The reference's tuner (lws/application/gpu/tune_launch.py:43-80) times every
candidate configuration of the raw and the fused kernel per (shape, batch),
keeps each kernel's fastest configuration that passes the accuracy check and
the best configuration shared by both (the order-matched one, AC-032), and
writes `tune-<gpu-slug>.json` (lws/adapters/filesystem/tuning_cache.py:
92-160; same JSON layout here, so files move both ways) - but nothing in the
reference loads that file back. Here `TuningFile.lookup` turns it into the
`launch_lookup` the runtime's layers call, and `load_packed` /
`load_reference` read it for the current GPU.

Candidates, the best and the order-matched rules are `se12_amd.launch`. The
GPU evaluator times one launch per sample after a read-only cache eviction
(median over samples, HIP events) and passes a configuration when its output
is within 1e-3 x max(|y|, 1) of a float32 torch product of the decoded
weights.

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
from typing import Callable, Iterable, Sequence

import torch

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


@dataclasses.dataclass(frozen=True)
class TuneRequest:
    rows: int
    cols: int
    batch: int


@dataclasses.dataclass(frozen=True)
class TunedEntry:
    rows: int
    cols: int
    batch: int
    raw: LaunchConfiguration
    fused: LaunchConfiguration
    order_matched: LaunchConfiguration


@dataclasses.dataclass(frozen=True)
class TuningFile:
    gpu_slug: str
    entries: tuple[TunedEntry, ...]

    def lookup(self, kind: str = "order_matched") -> Callable[[int, int, int], LaunchConfiguration | None]:
        """(rows, cols, batch) -> the tuned configuration of `kind`, or None
        (the library default) for a shape that was not tuned."""
        if kind not in KINDS:
            raise ValueError(f"kind must be one of {KINDS}")
        table = {(e.rows, e.cols, e.batch): getattr(e, kind) for e in self.entries}
        return lambda rows, cols, batch: table.get((rows, cols, batch))


def _cfg_to_json(c: LaunchConfiguration) -> dict:
    return {"threads_per_block": c.threads_per_block.value, "blocks": c.blocks.value}


def _cfg_from_json(d: dict) -> LaunchConfiguration:
    return LaunchConfiguration(ThreadsPerBlock(int(d["threads_per_block"])), BlockCount(int(d["blocks"])))


def to_json(tf: TuningFile) -> dict:
    return {"gpu_slug": tf.gpu_slug, "entries": [
        {"key": {"output_rows": e.rows, "k": e.cols, "batch": e.batch},
         "configurations": {"raw": _cfg_to_json(e.raw), "fused": _cfg_to_json(e.fused),
                            "order_matched": _cfg_to_json(e.order_matched)}} for e in tf.entries]}


def from_json(payload: dict) -> TuningFile:
    entries = []
    for raw in payload["entries"]:
        k, c = raw["key"], raw["configurations"]
        entries.append(TunedEntry(int(k["output_rows"]), int(k["k"]), int(k["batch"]), _cfg_from_json(c["raw"]),
                                  _cfg_from_json(c["fused"]), _cfg_from_json(c["order_matched"])))
    return TuningFile(payload["gpu_slug"], tuple(entries))


def tuning_directory(directory=None) -> pathlib.Path:
    if directory is not None:
        return pathlib.Path(directory)
    return pathlib.Path(os.environ.get("LWS_TUNING_DIR", "reports"))


def save_tuning(tf: TuningFile, directory=None) -> pathlib.Path:
    d = tuning_directory(directory)
    d.mkdir(parents=True, exist_ok=True)
    path = d / f"tune-{tf.gpu_slug}.json"
    path.write_text(json.dumps(to_json(tf), indent=2))
    return path


def load_tuning(gpu_slug: str, directory=None) -> TuningFile | None:
    """This GPU's tuning file, or None; files of other GPUs are ignored with a
    warning (tuning_cache.py:45-90)."""
    d = tuning_directory(directory)
    mine = d / f"tune-{gpu_slug}.json"
    if mine.exists():
        tf = from_json(json.loads(mine.read_text()))
        if tf.gpu_slug == gpu_slug:
            return tf
    for other in sorted(d.glob("tune-*.json")) if d.exists() else []:
        if other != mine:
            warnings.warn(f"ignoring {other}: tuned for another GPU (this one is {gpu_slug})")
    return None


Evaluator = Callable[[LaunchConfiguration], TimingAndAccuracy]


def tune_launch(gpu_slug: str, requests: Sequence[TuneRequest],
                evaluators: Callable[[TuneRequest], tuple[Evaluator, Evaluator]], directory=None,
                save: bool = True) -> TuningFile:
    """Times every candidate of both kernels per request (raw, fused) and keeps
    the fastest passing one of each and the best shared one; a request where
    nothing passes is left out (tune_launch.py:43-80)."""
    entries = []
    for req in requests:
        raw_eval, fused_eval = evaluators(req)
        cands = candidate_configurations(req.rows, req.cols, batch=req.batch)
        raw_timed = tuple(TimedCandidate(c, raw_eval(c)) for c in cands)
        fused_timed = tuple(TimedCandidate(c, fused_eval(c)) for c in cands)
        best_raw, best_fused = best_configuration(raw_timed), best_configuration(fused_timed)
        matched = order_matched_configuration(raw_timed, fused_timed)
        if best_raw is None or best_fused is None or matched is None:
            continue
        entries.append(TunedEntry(req.rows, req.cols, req.batch, best_raw, best_fused, matched))
    tf = TuningFile(gpu_slug, tuple(entries))
    if save:
        save_tuning(tf, directory)
    return tf


class GpuEvaluator:
    """Times one kernel's launches (median of `samples`, each after a cache
    eviction) and checks accuracy against a float32 product."""

    def __init__(self, kernel, x: torch.Tensor, reference: torch.Tensor, samples: int = 7, timer=None) -> None:
        from .hip import HipBenchmarkTimer

        self.kernel, self.x, self.ref = kernel, x, reference
        self.samples = samples
        self.timer = timer or HipBenchmarkTimer(x.device.index)
        self.scale = reference.abs().clamp_min(1.0)

    def __call__(self, cfg: LaunchConfiguration) -> TimingAndAccuracy:
        y = torch.empty((self.x.shape[0], self.kernel.rows), dtype=torch.float32, device=self.x.device)
        try:
            self.kernel.multiply(self.x, launch=cfg, out=y)
            torch.cuda.synchronize(self.x.device)
        except Exception:
            return TimingAndAccuracy(float("inf"), False)
        ok = bool(((y - self.ref).abs() / self.scale).max().item() <= 1e-3)
        st = self.timer.time_operation(lambda: self.kernel.multiply(self.x, launch=cfg, out=y), warmup=2,
                                       timed=self.samples)
        return TimingAndAccuracy(st.median_us, ok)


def gpu_evaluators(device, seed: int = 0, samples: int = 7):
    """Evaluators over random BF16 N(0, 0.02) weights of each requested shape
    (encoded on the GPU) and N(0, 1) activations."""
    from .hip import HipBenchmarkTimer, RawBf16MatVecKernel, Se12MatVecKernel, encode_on_device

    timer = HipBenchmarkTimer(torch.device(device).index)
    cache: dict = {}

    def make(req: TuneRequest):
        key = (req.rows, req.cols)
        if key not in cache:
            g = torch.Generator(device=device)
            g.manual_seed(seed + req.rows * 7 + req.cols)
            w = (torch.randn((req.rows, req.cols), generator=g, device=device) * 0.02).to(torch.bfloat16)
            cache[key] = (w, Se12MatVecKernel(encode_on_device(w)), RawBf16MatVecKernel(w))
        w, fused, raw = cache[key]
        g = torch.Generator(device=device)
        g.manual_seed(seed + 1 + req.batch)
        x = torch.randn((req.batch, req.cols), generator=g, device=device).to(torch.bfloat16)
        ref = x.float() @ w.float().t()
        return (GpuEvaluator(raw, x, ref, samples, timer), GpuEvaluator(fused, x, ref, samples, timer))

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
    reqs = [TuneRequest(int(s.split("x")[0]), int(s.split("x")[1]), int(b))
            for s in args.shapes.split(",") for b in args.batches.split(",")]
    slug = current_gpu_slug(dev)
    tf = tune_launch(slug, reqs, gpu_evaluators(dev, samples=args.samples), directory=args.out)
    print(f"tuning written for GPU '{slug}' ({len(tf.entries)} of {len(reqs)} (shape, batch) combinations) "
          f"in {tuning_directory(args.out) / f'tune-{slug}.json'}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
