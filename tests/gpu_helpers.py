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


def heavy_tailed_bf16_device(rows: int, cols: int, seed: int, device) -> torch.Tensor:
    """The same distribution as heavy_tailed_bf16, drawn on the GPU (numpy's
    Student-t takes about a minute at the LM head's 590 M weights): t(3) =
    z / sqrt(chi2_3 / 3) from four seeded normal draws, over sqrt(3) for
    unit variance, times 0.02; then about 0.1% of the entries (positions
    drawn with replacement) set to +-0.16. BF16 by round-to-nearest-even."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    t = torch.randn((rows, cols), generator=g, device=device)
    chi2 = torch.zeros_like(t)
    for _ in range(3):
        z = torch.randn((rows, cols), generator=g, device=device)
        chi2.addcmul_(z, z)
        del z
    t.mul_(torch.rsqrt(chi2.div_(3.0))).mul_(0.02 / 3.0 ** 0.5)
    del chi2
    n_out = max(1, rows * cols // 1000)
    pos = torch.randint(0, rows * cols, (n_out,), generator=g, device=device)
    sign = torch.randint(0, 2, (n_out,), generator=g, device=device).float() * 0.32 - 0.16
    t.view(-1)[pos] = sign
    return t.to(torch.bfloat16)


def uniform_bits(rows: int, cols: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.integers(0, 65536, size=(rows, cols), dtype=np.uint32).astype(np.uint16).view(np.int16)


# escape count of each tile of escape_count_bf16's matrix, tile-major
ESCAPE_COUNTS = (0, 1, 2, 7, 8, 9, 12, 16, 17, 3, 8, 9, 1, 16, 0, 5)


def escape_count_bf16(seed: int) -> tuple[np.ndarray, list[int]]:
    """A 64 x 1024 matrix (4 x 4 tiles) whose tiles hold exactly ESCAPE_COUNTS
    escapes: bulk exponents 111..125 fill the 15 codebook entries, each escape
    takes an exponent in 90..109. Positions include a tile's first and last
    weight, two escapes in one lane (16 weights) and every chunk. A tile with
    17 escapes exceeds the escape budget and is a fallback tile."""
    rng = np.random.default_rng(seed)
    e = rng.integers(111, 126, size=(64, 1024)).astype(np.uint16)
    for t, n in enumerate(ESCAPE_COUNTS):
        tr, tc = divmod(t, 4)
        if n == 0:
            continue
        fixed = [0, 4095, 17, 18][: min(n, 4)]        # first, last, two in lane 1 of chunk 0
        rest = rng.choice(np.setdiff1d(np.arange(4096), fixed), size=n - len(fixed), replace=False)
        pos = np.concatenate([np.array(fixed, dtype=np.int64), rest])
        e[tr * 16 + pos // 256, tc * 256 + pos % 256] = rng.integers(90, 110, size=n)
    sign = rng.integers(0, 2, size=e.shape).astype(np.uint16)
    mant = rng.integers(0, 0x80, size=e.shape).astype(np.uint16)
    return ((sign << 15) | (e << 7) | mant).view(np.int16), list(ESCAPE_COUNTS)

