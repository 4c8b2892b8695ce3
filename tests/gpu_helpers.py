"""Helpers shared by the GPU parity tests: oracle encodings uploaded to the
device, and the GEMV tolerance check."""

from __future__ import annotations

import numpy as np
import torch

from oracle import se12_codec as o
from se12_amd.format import Se12DeviceTensor, make_se12_tensor

# GEMV parity bound: |y - y_ref| <= REL_TOL * max(|y_ref|, 1), y_ref = the
# oracle's numpy decode + float32 matmul on the same inputs. 1e-3 relative is
# the bound the target sets; the max(., 1) clamp on the scale is the reference
# microbenchmark's (lws/bench/micro.py:154-159).
REL_TOL = 1e-3


def to_device(enc: dict, device) -> Se12DeviceTensor:
    rows, cols = enc["shape"]
    t = make_se12_tensor(enc["sm"], enc["ec"], enc["esc"], enc["fallback_bitmap"], enc["fallback_raw"],
                         enc["codebook"], rows, cols)
    return Se12DeviceTensor.from_host(t, device=device)


def bf16_tensor(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).astype(np.int16)).to(device).view(torch.bfloat16)


def max_rel_error(y: torch.Tensor, ref: np.ndarray) -> float:
    yy = y.detach().cpu().numpy().astype(np.float64)
    r = np.asarray(ref, dtype=np.float64)
    return float((np.abs(yy - r) / np.maximum(np.abs(r), 1.0)).max())


def normal_case(rows: int, cols: int, seed: int) -> tuple[np.ndarray, dict]:
    bits = o.normal_bf16(rows, cols, seed=seed, std=0.02)
    return bits, o.encode(bits.reshape(-1), rows, cols)


def heavy_tailed_bf16(rows: int, cols: int, seed: int) -> np.ndarray:
    """Student-t (df=3) scaled to std 0.02, 0.1% outliers at +-8 sigma."""
    rng = np.random.default_rng(seed)
    a = (rng.standard_t(3, size=(rows, cols)) / np.sqrt(3.0) * 0.02).astype(np.float32)
    n_out = max(1, rows * cols // 1000)
    idx = rng.choice(rows * cols, size=n_out, replace=False)
    a.reshape(-1)[idx] = np.where(rng.integers(0, 2, n_out) == 1, 0.16, -0.16).astype(np.float32)
    return o.f32_to_bf16_bits(a)


def uniform_bits(rows: int, cols: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.integers(0, 65536, size=(rows, cols), dtype=np.uint32).astype(np.uint16).view(np.int16)
