"""HIP adapters behind the reference's GPU ports, over libse12_gfx950.so.

  Se12MatVecKernel / RawBf16MatVecKernel  -> MatVecKernel
      (lws/application/ports/gpu/matvec_kernel.py:18-23,
       lws/adapters/cuda/gemv.py:143-226)
  HipSe12WeightDecoder                    -> WeightDecoder
      (lws/application/ports/gpu/weight_decoder.py:26-33,
       lws/adapters/cuda/se12_decoder.py:45-76)
  HipGpuProbe                             -> GpuProbe
      (lws/application/ports/gpu/gpu_probe.py:17-27)
  HipBenchmarkTimer                       -> BenchmarkTimer
      (lws/application/ports/gpu/benchmark_timer.py:13-21)
  encode_on_device                        -> the packer's encode_tensor step
      (lws/domain/se12/codec.py:111-141), run on the GPU

Torch is used only to own device memory and to name the stream; every kernel
is launched by the library on the caller's current HIP stream.
"""

from __future__ import annotations

import ctypes
import dataclasses
import os
import statistics as _st
from typing import Any, Callable

import numpy as np
import torch

from . import _native as nat
from .format import (
    CODEBOOK_SIZE,
    ESCAPE_BUDGET,
    TILE_SIZE,
    Bf16Weights,
    Se12DeviceTensor,
    bitmap_bytes,
    tile_grid,
    validate_device_streams,
)
from . import ports as P
from .launch import BlockCount, LaunchConfiguration, ThreadsPerBlock


def _device_of(t: torch.Tensor) -> torch.device:
    if not t.is_cuda:
        raise ValueError("expected a tensor on a HIP device")
    return t.device


def _as_device_tensor(tensor: Any, device=None) -> Se12DeviceTensor:
    if isinstance(tensor, Se12DeviceTensor):
        validate_device_streams(tensor)
        if device is not None and tensor.sm.device != torch.device(device):
            raise ValueError(f"SE12 streams on {tensor.sm.device}, requested {device}")
        return tensor
    return Se12DeviceTensor.from_host(tensor, device=device)


def _require(t: Any, name: str, dtype: torch.dtype, shape: tuple, device: torch.device) -> torch.Tensor:
    """Checks a caller-supplied tensor before its pointer crosses into the
    library: a host tensor, another device's memory or a short buffer would
    otherwise reach a kernel as a bad address."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch tensor, got {type(t).__name__}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, the weights on {device}")
    if t.dtype != dtype or tuple(t.shape) != tuple(shape) or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dtype} {list(shape)} tensor, "
                         f"got {t.dtype} {list(t.shape)}{'' if t.is_contiguous() else ' (not contiguous)'}")
    return t


class _Handle:
    """Owns one se12_handle*; released when garbage-collected."""

    def __init__(self, raw: ctypes.c_void_p, keepalive: tuple) -> None:
        self.raw = raw
        self._keepalive = keepalive  # the tensors the handle points into

    def release(self) -> None:
        if self.raw:
            nat.lib().se12_release(self.raw)
            self.raw = ctypes.c_void_p(None)

    def __del__(self) -> None:
        try:
            self.release()
        except Exception:
            pass

    def default_launch(self, batch: int) -> LaunchConfiguration:
        out = nat.Launch()
        nat.check(nat.lib().se12_default_launch(self.raw, batch, ctypes.byref(out)))
        return LaunchConfiguration(ThreadsPerBlock(out.threads_per_block), BlockCount(out.blocks))


def bind_se12(dt: Se12DeviceTensor, max_batch: int = nat.MAX_BATCH) -> _Handle:
    s = nat.Streams(
        sm_dev=dt.sm.data_ptr(),
        ec_dev=dt.ec.data_ptr(),
        esc_dev=dt.esc.data_ptr(),
        codebook_dev=dt.codebook.data_ptr(),
        fallback_bitmap_dev=dt.fallback_bitmap.data_ptr(),
        fallback_raw_dev=dt.fallback_raw.data_ptr() if dt.fallback_raw.numel() else None,
        fallback_raw_elems=int(dt.fallback_raw.numel()),
    )
    h = ctypes.c_void_p()
    with torch.cuda.device(dt.sm.device):
        nat.check(nat.lib().se12_bind(ctypes.byref(s), dt.rows, dt.cols, max_batch, nat.stream_ptr(), ctypes.byref(h)))
    return _Handle(h, (dt,))


def bind_raw_bf16(w: torch.Tensor, max_batch: int = nat.MAX_BATCH) -> _Handle:
    if w.dtype != torch.bfloat16 or w.dim() != 2:
        raise ValueError("raw twin needs a 2-D bfloat16 weight matrix")
    w = w.contiguous()
    h = ctypes.c_void_p()
    with torch.cuda.device(w.device):
        nat.check(nat.lib().se12_bind_raw_bf16(nat.ptr(w), w.shape[0], w.shape[1], max_batch, nat.stream_ptr(), ctypes.byref(h)))
    return _Handle(h, (w,))


def _launch_struct(launch: LaunchConfiguration | None):
    if launch is None:
        return None
    return ctypes.byref(nat.Launch(launch.threads_per_block.value, launch.blocks.value))


class _GemvBase:
    rows: int
    cols: int
    handle: _Handle
    device: torch.device

    def multiply(self, activations: torch.Tensor, launch: LaunchConfiguration | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """y = x . W^T in FP32 for x [B, K] (BF16 or FP32) on the device;
        `launch=None` uses the default configuration (matvec_kernel.py:19-22)."""
        x = activations
        if x.dim() == 1:
            x = x.unsqueeze(0)
        if x.dim() != 2 or x.shape[1] != self.cols:
            raise ValueError(f"activations must be [B, {self.cols}], got {tuple(activations.shape)}")
        if x.device != self.device:
            raise ValueError(f"activations on {x.device}, weights on {self.device}")
        if x.dtype == torch.bfloat16:
            xd = nat.X_BF16
        elif x.dtype == torch.float32:
            xd = nat.X_F32
        else:
            raise ValueError(f"activations must be bfloat16 or float32, got {x.dtype}")
        x = x.contiguous()
        b = x.shape[0]
        out = _fp32_out(out, b, self.rows, self.device)
        nat.check(nat.lib().se12_gemv(self.handle.raw, nat.ptr(x), xd, b, nat.ptr(out), _launch_struct(launch), nat.stream_ptr()))
        return out

    def default_launch(self, batch: int) -> LaunchConfiguration:
        return self.handle.default_launch(batch)

    def multiply_noalloc(self, activations: torch.Tensor, out: torch.Tensor,
                         launch: LaunchConfiguration | None = None) -> torch.Tensor:
        """`multiply` through se12_gemv_noalloc: the library allocates nothing
        (its split-K scratch is a static per-GPU array shared by every such
        call on the GPU, so overlapping calls race); `out` is required, and
        x must be contiguous (it is not copied)."""
        x, xd = _activations(activations, self.cols, self.device, copy=False)
        out = _require(out, "out", torch.float32, (x.shape[0], self.rows), self.device)
        nat.check(nat.lib().se12_gemv_noalloc(self.handle.raw, nat.ptr(x), xd, x.shape[0], nat.ptr(out),
                                              _launch_struct(launch), nat.stream_ptr()))
        return out

    def multiply_rmsnorm(self, activations: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, residual: torch.Tensor,
                         out: torch.Tensor, eps: float, y: torch.Tensor | None = None,
                         launch: LaunchConfiguration | None = None) -> torch.Tensor:
        """y = x . W^T (FP32, as `multiply`), then per batch row the decoder's
        post-norm, residual add and next pre-norm in the product's tail:
        residual = bf16(residual + norm(bf16(y)) * (1 + w1)),
        out = norm(residual) * (1 + w2), norm(t) = t * rsqrt(mean(t^2) + eps).
        residual / out: BF16 [B, rows] (updated / written); returns y."""
        x, xd = _activations(activations, self.cols, self.device)
        b = x.shape[0]
        y = _fp32_out(y, b, self.rows, self.device, "y")
        for name, t in (("w1", w1), ("w2", w2)):
            _require(t, name, torch.bfloat16, (self.rows,), self.device)
        for name, t in (("residual", residual), ("out", out)):
            _require(t, name, torch.bfloat16, (b, self.rows), self.device)
        nat.check(nat.lib().se12_gemv_rmsnorm(self.handle.raw, nat.ptr(x), xd, b, nat.ptr(y), nat.ptr(w1), nat.ptr(w2),
                                              nat.ptr(residual), nat.ptr(out), float(eps), _launch_struct(launch),
                                              nat.stream_ptr()))
        return y

    def multiply_rowss(self, activations: torch.Tensor, row_ss: torch.Tensor, y: torch.Tensor | None = None,
                       launch: LaunchConfiguration | None = None) -> torch.Tensor:
        """y = x . W^T with the tile-row sums of squares of the output
        (se12_gemv_rowss): row_ss[b, t] = sum over tile row t's 16 rows of
        bf16(y[b, n])^2, FP32 [B, ceil(rows / 16)], for a following
        `multiply_prenorm(..., y_prev_ss=row_ss)`. Returns y."""
        x, xd = _activations(activations, self.cols, self.device)
        b = x.shape[0]
        y = _fp32_out(y, b, self.rows, self.device, "y")
        _require(row_ss, "row_ss", torch.float32, (b, (self.rows + 15) // 16), self.device)
        nat.check(nat.lib().se12_gemv_rowss(self.handle.raw, nat.ptr(x), xd, b, nat.ptr(y), nat.ptr(row_ss),
                                            _launch_struct(launch), nat.stream_ptr()))
        return y


class Se12MatVecKernel(_GemvBase):
    """Fused SE12 decode + GEMV bound to one SE12 matrix (gemv.py:180-226).

    `tensor` is a host `Se12Tensor` (reference layout, uploaded once) or an
    `Se12DeviceTensor` already in HBM."""

    def __init__(self, tensor: Any, max_batch: int = nat.MAX_BATCH, device=None) -> None:
        self.tensor = _as_device_tensor(tensor, device)
        self.rows, self.cols = self.tensor.rows, self.tensor.cols
        self.device = self.tensor.sm.device
        self.handle = bind_se12(self.tensor, max_batch)

    def bind_stats(self) -> dict:
        """What bind derived (se12_handle_bind_stats): `raw_tiles`, the tiles
        decoded once to raw BF16 because they hold more escapes than a side
        record lists (the kernels read their 8,192 raw bytes besides the
        tile's streams), and `sidecar_bytes`, the device bytes of the
        derived data."""
        raw, side = ctypes.c_int64(), ctypes.c_int64()
        nat.check(nat.lib().se12_handle_bind_stats(self.handle.raw, ctypes.byref(raw), ctypes.byref(side)))
        return {"raw_tiles": int(raw.value), "sidecar_bytes": int(side.value)}

    def decode_into(self, out: torch.Tensor) -> torch.Tensor:
        """Decodes the whole matrix into `out` (row-major BF16 [rows, cols],
        e.g. a view of a scratch buffer shared by many layers)."""
        _require(out, "out", torch.bfloat16, (self.rows, self.cols), self.device)
        nat.check(nat.lib().se12_decode(self.handle.raw, nat.ptr(out), nat.stream_ptr()))
        return out

    def decode_rows_into(self, rows: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """Decodes the rows of a device int64 index tensor, in order, into `out`
        ([len(rows), cols] BF16); only the tiles of those rows are read. An
        index outside [0, rows) gives a row of zeros (the kernel checks each
        index before reading)."""
        idx = rows.reshape(-1)
        _require(idx, "rows", torch.int64, (idx.numel(),), self.device)
        _require(out, "out", torch.bfloat16, (idx.numel(), self.cols), self.device)
        nat.check(nat.lib().se12_decode_rows(self.handle.raw, nat.ptr(idx), idx.numel(), nat.ptr(out), nat.stream_ptr()))
        return out


class RawBf16MatVecKernel(_GemvBase):
    """The same-skeleton raw-BF16 twin bound to a [N, K] BF16 matrix (gemv.py:143-172)."""

    def __init__(self, weights: torch.Tensor, max_batch: int = nat.MAX_BATCH) -> None:
        self.weights = weights.contiguous()
        self.rows, self.cols = self.weights.shape
        self.device = _device_of(self.weights)
        self.handle = bind_raw_bf16(self.weights, max_batch)


def _activations(activations: torch.Tensor, cols: int, device, copy: bool = True) -> tuple[torch.Tensor, int]:
    """x as a contiguous [B, cols] tensor and its library dtype code. With
    `copy=False` a non-contiguous x is refused instead of copied (the copy is
    a device allocation)."""
    x = activations.unsqueeze(0) if activations.dim() == 1 else activations
    if x.dim() != 2 or x.shape[1] != cols:
        raise ValueError(f"activations must be [B, {cols}], got {tuple(activations.shape)}")
    if x.device != device:
        raise ValueError(f"activations on {x.device}, weights on {device}")
    if x.dtype == torch.bfloat16:
        code = nat.X_BF16
    elif x.dtype == torch.float32:
        code = nat.X_F32
    else:
        raise ValueError(f"activations must be bfloat16 or float32, got {x.dtype}")
    if not x.is_contiguous():
        if not copy:
            raise ValueError("activations must be contiguous here: copying them would allocate device memory")
        x = x.contiguous()
    return x, code


def _fp32_out(out: torch.Tensor | None, b: int, rows: int, device, name: str = "out") -> torch.Tensor:
    if out is None:
        return torch.empty((b, rows), dtype=torch.float32, device=device)
    return _require(out, name, torch.float32, (b, rows), device)


def multiply_gelu_mul(gate, up, activations: torch.Tensor, out: torch.Tensor, ys: list[torch.Tensor] | None = None,
                      launch: LaunchConfiguration | None = None) -> list[torch.Tensor]:
    """The grouped product of two bound matrices with the same rows (the MLP's
    gate and up), then out = bf16(gelu_tanh(bf16(y_gate)) * bf16(y_up)) in the
    product's tail. out: BF16 [B, rows]; returns the FP32 [y_gate, y_up]."""
    if gate.rows != up.rows or gate.cols != up.cols or gate.device != up.device or type(gate) is not type(up):
        raise ValueError("gate and up need one shape, one device and one format")
    x, xd = _activations(activations, gate.cols, gate.device)
    b = x.shape[0]
    if ys is not None and len(ys) != 2:
        raise ValueError(f"ys must hold two tensors, got {len(ys)}")
    ys = [_fp32_out(None if ys is None else ys[i], b, gate.rows, gate.device, f"ys[{i}]") for i in range(2)]
    _require(out, "out", torch.bfloat16, (b, gate.rows), gate.device)
    hs = (ctypes.c_void_p * 2)(gate.handle.raw.value, up.handle.raw.value)
    yp = (ctypes.c_void_p * 2)(ys[0].data_ptr(), ys[1].data_ptr())
    nat.check(nat.lib().se12_gemv_gelu_mul(hs, nat.ptr(x), xd, b, yp, nat.ptr(out), _launch_struct(launch),
                                           nat.stream_ptr()))
    return ys


def multiply_prenorm(kernels, y_prev: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, residual_in: torch.Tensor,
                     residual_out: torch.Tensor, h_out: torch.Tensor, eps: float, ys: list[torch.Tensor] | None = None,
                     gelu_out: torch.Tensor | None = None, launch: LaunchConfiguration | None = None,
                     y_prev_ss: torch.Tensor | None = None) -> list[torch.Tensor]:
    """The decoder's next normalised input and its products in one launch
    (se12_gemv_prenorm): per batch row of the previous product's FP32 output
    y_prev [B, K], r = bf16(residual_in + norm(bf16(y_prev)) * (1 + w1)),
    h = norm(r) * (1 + w2); residual_out = r, h_out = h, then y_i = h . W_i^T
    for up to 4 bound matrices with K columns (and, with gelu_out and two
    matrices, the MLP gate of `multiply_gelu_mul`). residual_in and
    residual_out are the same tensor or disjoint. y_prev_ss: the row sums that
    `multiply_rowss` wrote with y_prev (the first norm's mean then comes from
    them). Returns the FP32 y_i."""
    kernels = list(kernels)
    if not 1 <= len(kernels) <= nat.MAX_GROUP:
        raise ValueError(f"1..{nat.MAX_GROUP} matrices per launch, got {len(kernels)}")
    k0 = kernels[0]
    for k in kernels:
        if k.cols != k0.cols or k.device != k0.device or type(k) is not type(k0):
            raise ValueError("the matrices need one K, one device and one format")
    if not isinstance(y_prev, torch.Tensor) or y_prev.dim() != 2:
        raise ValueError(f"y_prev must be a 2-D float32 [B, {k0.cols}] tensor")
    b = y_prev.shape[0]
    _require(y_prev, "y_prev", torch.float32, (b, k0.cols), k0.device)
    if y_prev_ss is not None:
        _require(y_prev_ss, "y_prev_ss", torch.float32, (b, (k0.cols + 15) // 16), k0.device)
    for name, t in (("w1", w1), ("w2", w2)):
        _require(t, name, torch.bfloat16, (k0.cols,), k0.device)
    for name, t in (("residual_in", residual_in), ("residual_out", residual_out), ("h_out", h_out)):
        _require(t, name, torch.bfloat16, (b, k0.cols), k0.device)
    if ys is not None and len(ys) != len(kernels):
        raise ValueError(f"ys must hold {len(kernels)} tensors, got {len(ys)}")
    ys = [_fp32_out(None if ys is None else ys[i], b, k.rows, k0.device, f"ys[{i}]") for i, k in enumerate(kernels)]
    if gelu_out is not None:
        if len(kernels) != 2 or kernels[0].rows != kernels[1].rows:
            raise ValueError("the MLP gate takes two matrices with the same rows")
        _require(gelu_out, "gelu_out", torch.bfloat16, (b, k0.rows), k0.device)
    n = len(kernels)
    hs = (ctypes.c_void_p * n)(*[k.handle.raw.value for k in kernels])
    yp = (ctypes.c_void_p * n)(*[t.data_ptr() for t in ys])
    nat.check(nat.lib().se12_gemv_prenorm(hs, n, nat.ptr(y_prev),
                                          None if y_prev_ss is None else nat.ptr(y_prev_ss), b, nat.ptr(w1), nat.ptr(w2), nat.ptr(residual_in),
                                          nat.ptr(residual_out), nat.ptr(h_out), float(eps), yp,
                                          None if gelu_out is None else nat.ptr(gelu_out), _launch_struct(launch),
                                          nat.stream_ptr()))
    return ys


def multiply_grouped(kernels, activations: torch.Tensor, launch: LaunchConfiguration | None = None,
                     outs: list[torch.Tensor] | None = None) -> list[torch.Tensor]:
    """y_i = x . W_i^T for up to 4 bound matrices with the same K (e.g. q, k, v
    or gate, up) in one launch; all of one format (fused SE12 or raw twin).
    `launch` counts the matrices' tile rows together (blocks = their sum x K
    splits). Outputs equal separate `multiply` calls under the same waves per
    block and K splits."""
    kernels = list(kernels)
    if not 1 <= len(kernels) <= nat.MAX_GROUP:
        raise ValueError(f"1..{nat.MAX_GROUP} matrices per grouped launch, got {len(kernels)}")
    k0 = kernels[0]
    x = activations.unsqueeze(0) if activations.dim() == 1 else activations
    for k in kernels:
        if k.cols != k0.cols or k.device != k0.device or type(k) is not type(k0):
            raise ValueError("grouped matrices need one K, one device and one format")
    if x.dim() != 2 or x.shape[1] != k0.cols:
        raise ValueError(f"activations must be [B, {k0.cols}], got {tuple(activations.shape)}")
    if x.device != k0.device:
        raise ValueError(f"activations on {x.device}, weights on {k0.device}")
    if x.dtype == torch.bfloat16:
        xd = nat.X_BF16
    elif x.dtype == torch.float32:
        xd = nat.X_F32
    else:
        raise ValueError(f"activations must be bfloat16 or float32, got {x.dtype}")
    x = x.contiguous()
    b = x.shape[0]
    if outs is not None and len(outs) != len(kernels):
        raise ValueError(f"outs must hold {len(kernels)} tensors, got {len(outs)}")
    outs = [_fp32_out(None if outs is None else outs[i], b, k.rows, k0.device, f"outs[{i}]")
            for i, k in enumerate(kernels)]
    n = len(kernels)
    hs = (ctypes.c_void_p * n)(*[k.handle.raw.value for k in kernels])
    ys = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    nat.check(nat.lib().se12_gemv_grouped(hs, n, nat.ptr(x), xd, b, ys, _launch_struct(launch), nat.stream_ptr()))
    return outs


@dataclasses.dataclass(frozen=True)
class RowIndices:
    """Row indices in request order (weight_decoder.py:18-23)."""

    values: tuple[int, ...]


class HipSe12WeightDecoder:
    """WeightDecoder on the GPU (se12_decoder.py:45-76). Bindings are cached per
    device tensor so repeated decodes reuse the bind-time sidecar."""

    def __init__(self) -> None:
        self._last: tuple[Any, Se12DeviceTensor, _Handle] | None = None

    def _handle(self, tensor: Any) -> tuple[Se12DeviceTensor, _Handle]:
        if self._last is not None and self._last[0] is tensor:
            return self._last[1], self._last[2]
        dt = _as_device_tensor(tensor)
        h = bind_se12(dt, max_batch=1)
        self._last = (tensor, dt, h)
        return dt, h

    def decode_to_device(self, tensor: Any) -> torch.Tensor:
        """Decoded weights as a device BF16 [rows, cols] tensor (se12_decoder.py:58-62)."""
        dt, h = self._handle(tensor)
        out = torch.empty((dt.rows, dt.cols), dtype=torch.bfloat16, device=dt.sm.device)
        nat.check(nat.lib().se12_decode(h.raw, nat.ptr(out), nat.stream_ptr()))
        return out

    def decode(self, tensor: Any) -> Bf16Weights:
        """Host copy of the decoded bit pattern (se12_decoder.py:54-56)."""
        out = self.decode_to_device(tensor)
        return Bf16Weights(bit_pattern=out.view(torch.int16).cpu().numpy().reshape(-1))

    def decode_rows_to_device(self, tensor: Any, rows: torch.Tensor) -> torch.Tensor:
        """Rows given by a device int64 index tensor, in order; only their tiles are read."""
        dt, h = self._handle(tensor)
        idx = rows.to(device=dt.sm.device, dtype=torch.int64).contiguous()
        out = torch.empty((idx.numel(), dt.cols), dtype=torch.bfloat16, device=dt.sm.device)
        nat.check(nat.lib().se12_decode_rows(h.raw, nat.ptr(idx), idx.numel(), nat.ptr(out), nat.stream_ptr()))
        return out

    def decode_rows(self, tensor: Any, rows: RowIndices) -> Bf16Weights:
        """The decoded rows, in request order (weight_decoder.py:30-33)."""
        dt, _ = self._handle(tensor)
        values = tuple(int(r) for r in rows.values)
        bad = [r for r in values if not 0 <= r < dt.rows]
        if bad:
            raise IndexError(f"row indices {bad[:4]} outside [0, {dt.rows})")
        idx = torch.tensor(values, dtype=torch.int64, device=dt.sm.device)
        out = self.decode_rows_to_device(tensor, idx)
        return Bf16Weights(bit_pattern=out.view(torch.int16).cpu().numpy().reshape(-1))


def encode_on_device(weights: torch.Tensor) -> Se12DeviceTensor:
    """SE12-encodes a [rows, cols] BF16 device tensor on the GPU; the streams are
    byte-identical to the reference encoder's (codec.py:111-141)."""
    if weights.dtype != torch.bfloat16 or weights.dim() != 2:
        raise ValueError("encode_on_device needs a 2-D bfloat16 tensor")
    w = weights.contiguous()
    dev = _device_of(w)
    rows, cols = w.shape
    tr, tc = tile_grid(rows, cols)
    t = tr * tc
    cb = (ctypes.c_uint8 * CODEBOOK_SIZE)()
    nfb = ctypes.c_int64()
    lib = nat.lib()
    with torch.cuda.device(dev):
        st = nat.stream_ptr()
        nat.check(lib.se12_encode_prepare(nat.ptr(w), rows, cols, cols, cb, ctypes.byref(nfb), st))
        sm = torch.empty(t * TILE_SIZE, dtype=torch.uint8, device=dev)
        ec = torch.empty(t * TILE_SIZE // 2, dtype=torch.uint8, device=dev)
        esc = torch.empty(t * ESCAPE_BUDGET, dtype=torch.uint8, device=dev)
        bitmap = torch.empty(bitmap_bytes(t), dtype=torch.uint8, device=dev)
        raw = torch.empty(nfb.value * TILE_SIZE, dtype=torch.int16, device=dev)
        out = nat.StreamsOut(
            sm_dev=sm.data_ptr(), ec_dev=ec.data_ptr(), esc_dev=esc.data_ptr(), fallback_bitmap_dev=bitmap.data_ptr(),
            fallback_raw_dev=raw.data_ptr() if raw.numel() else None, fallback_raw_tiles=nfb.value,
        )
        got = ctypes.c_int64()
        nat.check(lib.se12_encode(nat.ptr(w), rows, cols, cols, cb, ctypes.byref(out), ctypes.byref(got), st))
    codebook = tuple(int(c) for c in cb)
    return Se12DeviceTensor(
        sm=sm, ec=ec, esc=esc, codebook=torch.tensor(codebook, dtype=torch.uint8, device=dev),
        fallback_bitmap=bitmap, fallback_raw=raw, rows=int(rows), cols=int(cols), codebook_host=codebook,
    )


def codebook_from_histogram(counts) -> tuple[int, ...]:
    """Host call into the library's codebook rule (codebook.py:41-59)."""
    arr = (ctypes.c_uint64 * 256)(*[int(c) for c in counts])
    out = (ctypes.c_uint8 * CODEBOOK_SIZE)()
    nat.check(nat.lib().se12_codebook_from_histogram(arr, out))
    return tuple(int(c) for c in out)


# ---------------------------------------------------------------------------
# device facts and timing
# ---------------------------------------------------------------------------


HBM_TRANSFERS_PER_CLOCK = 4
DEVICE_INDEX_ENV_VAR = "LWS_DEVICE"


@dataclasses.dataclass(frozen=True)
class DeviceFacts:
    """hipDeviceProp_t facts the roofline, the launch heuristic and the
    reports use (flat; the port's nested DeviceProperties is built from it)."""

    name: str
    arch: str
    compute_units: int
    wavefront_size: int
    l2_bytes: int
    lds_bytes_per_cu: int
    lds_bytes_per_block: int
    total_memory_bytes: int
    clock_khz: int
    memory_clock_khz: int
    memory_bus_width_bits: int
    pci_domain_id: int = 0
    pci_bus_id: int = 0
    pci_device_id: int = 0
    ecc_enabled: bool = False
    kernel_timeout: bool = False
    runtime_version: int = 0
    driver_version: int = 0

    @property
    def pci_address(self) -> str:
        """"dddd:bb:dd.0", the device's PCI location (sysfs naming)."""
        return f"{self.pci_domain_id:04x}:{self.pci_bus_id:02x}:{self.pci_device_id:02x}.0"

    @property
    def hbm_peak_gbps(self) -> float:
        """Peak HBM bandwidth from hipDeviceProp's memory clock and bus width.
        HBM3 / HBM3E move HBM_TRANSFERS_PER_CLOCK data words per pin per
        reported clock: MI355X reports 2.0 GHz on an 8192-bit interface,
        i.e. 8 Gb/s per pin, 8,192 GB/s (the published peak is 8.0 TB/s)."""
        return self.memory_clock_khz * 1e3 * HBM_TRANSFERS_PER_CLOCK * self.memory_bus_width_bits / 8.0 / 1e9

    @property
    def slug(self) -> str:
        """GPU slug for per-GPU files, e.g. 'amd-instinct-mi355x-gfx950'."""
        base = "".join(ch.lower() if ch.isalnum() else "-" for ch in self.name).strip("-")
        while "--" in base:
            base = base.replace("--", "-")
        return f"{base}-{self.arch.split(':')[0]}"

    @property
    def capability(self) -> tuple[int, int]:
        """(major, minor) of the gfx architecture as HIP reports them
        (hipDeviceProp major / minor): gfx950 -> (9, 5), gfx942 -> (9, 4)."""
        digits = self.arch.split(":")[0].removeprefix("gfx")
        return int(digits[:-2] or 0), int(digits[-2], 16) if len(digits) >= 2 else 0


def _library_targets() -> tuple[int, ...]:
    """The architectures the library holds code objects for, in the
    capability encoding (major * 10 + minor: gfx950 -> 95)."""
    from .compiler import LIBRARY_ARCHES, arch_number

    return tuple(arch_number(a) for a in LIBRARY_ARCHES)


class HipGpuProbe:
    """GpuProbe over hipGetDeviceProperties (lws/application/ports/gpu/
    gpu_probe.py:17-27, the reference adapter lws/adapters/cuda/gpu_probe.py:
    59-80): `properties()`, `software_versions()` and `smoke_test()` return
    the port's value objects (se12_amd.ports); `facts()` the flat
    hipDeviceProp_t record this package's own code reads."""

    def __init__(self, device: int | None = None) -> None:
        if device is None:
            env = os.environ.get(DEVICE_INDEX_ENV_VAR)  # the reference's default (gpu_probe.py:83-89)
            device = int(env) if env is not None else torch.cuda.current_device()
        self.device = device

    def facts(self) -> DeviceFacts:
        info = nat.DeviceInfo()
        nat.check(nat.lib().se12_device_info_get(self.device, ctypes.byref(info)))
        return DeviceFacts(
            name=info.name.decode(), arch=info.arch.decode(), compute_units=info.compute_units,
            wavefront_size=info.wavefront_size, l2_bytes=info.l2_bytes, lds_bytes_per_cu=info.lds_bytes_per_cu,
            lds_bytes_per_block=info.lds_bytes_per_block, total_memory_bytes=info.total_memory_bytes,
            clock_khz=info.clock_khz, memory_clock_khz=info.memory_clock_khz,
            memory_bus_width_bits=info.memory_bus_width_bits, pci_domain_id=info.pci_domain_id,
            pci_bus_id=info.pci_bus_id, pci_device_id=info.pci_device_id, ecc_enabled=bool(info.ecc_enabled),
            kernel_timeout=bool(info.kernel_timeout), runtime_version=info.runtime_version,
            driver_version=info.driver_version,
        )

    def properties(self) -> P.DeviceProperties:
        """The nested DeviceProperties the reference's entry points read
        (lws/domain/device/properties.py:98-107): identity and slug, compute
        units as `sm_count`, VRAM total / free, L2 size, peak bandwidth from
        the memory clock, and the library's code-object targets."""
        f = self.facts()
        free, total = torch.cuda.mem_get_info(self.device)
        major, minor = f.capability
        identity = P.DeviceIdentity(name=P.DeviceName(f.name), slug=P.GpuSlug(f.slug))
        compute = P.ComputeHardware(capability=P.ComputeCapability(major=major, minor=minor),
                                    sm_count=P.SmCount(f.compute_units))
        memory = P.MemoryProfile(
            vram=P.VramSizes(total=P.Bytes(int(total)), free=P.Bytes(int(free))),
            characteristics=P.MemoryCharacteristics(l2_size=P.Bytes(f.l2_bytes),
                                                    bandwidth=P.GigabytesPerSecond(f.hbm_peak_gbps)))
        return P.DeviceProperties(
            identity_and_compute=P.IdentityAndCompute(identity=identity, compute=compute),
            memory_and_nvrtc=P.MemoryAndNvrtc(memory=memory, nvrtc_targets=P.NvrtcTargets(_library_targets())))

    def software_versions(self) -> P.SoftwareVersions:
        """Report-only versions (properties.py:147-165): HIP driver and
        runtime, torch and its architecture list, the library's build string
        in CuPy's and NVRTC's places."""
        f = self.facts()
        lib_version = nat.version()
        arch_list = tuple(torch.cuda.get_arch_list()) if hasattr(torch.cuda, "get_arch_list") else ()
        core = P.VersionsCore(
            toolchain=P.ToolchainVersions(driver=str(f.driver_version), cuda_runtime=str(f.runtime_version)),
            torch_and_cupy=P.TorchAndCupy(torch=P.TorchInfo(version=torch.__version__,
                                                            arch_list=P.TorchArchList(arch_list)),
                                          cupy_version=lib_version))
        return P.SoftwareVersions(core=core, nvrtc=P.NvrtcInfo(version=lib_version,
                                                              targets=P.NvrtcTargets(_library_targets())))

    def smoke_test(self) -> P.SupportVerdict:
        """Does torch run a kernel on this device, and does the library's
        kernel (one 16 x 256 fused product) give the right sum (the reference's
        check, gpu_probe.py:152-166, runs a torch kernel only)."""
        try:
            dev = torch.device("cuda", self.device)
            a = torch.full((8,), 1.0, device=dev) * 2
            if a.sum().item() != 16.0:
                return P.SupportVerdict(False)
            w = torch.full((16, 256), 1.0, dtype=torch.bfloat16, device=dev)
            x = torch.full((1, 256), 0.5, dtype=torch.bfloat16, device=dev)
            y = Se12MatVecKernel(encode_on_device(w), max_batch=1).multiply(x)
            return P.SupportVerdict(bool(torch.all(y == 128.0).item()))
        except Exception:
            return P.SupportVerdict(False)


# MI355X's last-level Infinity Cache (MALL) is not reported by hipDeviceProp;
# the flush covers it explicitly.
INFINITY_CACHE_BYTES = 256 * 1024 * 1024
GIBIBYTE = 1024 ** 3
PEAK_COPY_FRACTION_OF_FREE = 0.25


@dataclasses.dataclass(frozen=True)
class LatencyStats:
    median_us: float
    p10_us: float
    p90_us: float
    samples: tuple[float, ...]


def latency_stats(samples_us) -> LatencyStats:
    arr = np.asarray(samples_us, dtype=np.float64)
    return LatencyStats(float(np.median(arr)), float(np.percentile(arr, 10)), float(np.percentile(arr, 90)), tuple(arr.tolist()))


class HipBenchmarkTimer:
    """BenchmarkTimer (lws/application/ports/gpu/benchmark_timer.py:13-21):
    HIP event timing after a cache eviction of at least 2 x (L2 + Infinity
    Cache) (the reference adapter, lws/adapters/cuda/benchmark_timer.py:
    20-66, flushes 2 x L2 only). Constructed as the reference's
    `CudaBenchmarkTimer(device_index, l2_size)`; `l2_size` is a `Bytes`-like
    object or an int, queried from the device when omitted.

    Port methods: `time_operation(operation, counts) -> LatencySamples` and
    `measure_peak_copy_bandwidth() -> GigabytesPerSecond`. The package's own
    measurements use `time_stats`, `time_cold_rotation` and
    `measure_copy_traffic_gbps`."""

    def __init__(self, device_index: int | None = None, l2_size: Any = None) -> None:
        self.device = torch.cuda.current_device() if device_index is None else int(device_index)
        if l2_size is None:
            l2_size = HipGpuProbe(self.device).facts().l2_bytes
        self.l2_size = int(P.value_of(l2_size))
        flush = 2 * (self.l2_size + INFINITY_CACHE_BYTES)
        self.flush_buffer = torch.zeros(flush // 4, dtype=torch.float32, device=f"cuda:{self.device}")

    def flush(self) -> None:
        """Evicts by reading the buffer: a fill would leave the caches full of
        dirty lines whose write-back competes with the timed operation."""
        torch.sum(self.flush_buffer)

    # -- the port --------------------------------------------------------

    def time_operation(self, operation: Callable[[], Any], counts: Any) -> P.LatencySamples:
        """`counts.warmup` untimed runs, then `counts.timed` samples, each
        after a cache eviction, in microseconds (benchmark_timer.py:31-50)."""
        st = self.time_stats(operation, warmup=int(counts.warmup), timed=int(counts.timed))
        return P.LatencySamples(values=st.samples)

    def measure_peak_copy_bandwidth(self) -> P.GigabytesPerSecond:
        """GB/s of a device-to-device FP32 copy of min(1 GiB, 25% of free
        memory), the copied bytes counted once, median of 20 samples after 10
        warmups: the reference's peak (benchmark_timer.py:55-66), which its
        verdict's 70% bar divides by."""
        free, _ = torch.cuda.mem_get_info(self.device)
        target = min(GIBIBYTE, int(free * PEAK_COPY_FRACTION_OF_FREE))
        n = -(-target // 4)
        src = torch.empty(n, dtype=torch.float32, device=f"cuda:{self.device}")
        dst = torch.empty_like(src)
        st = self.time_stats(lambda: dst.copy_(src), warmup=10, timed=20)
        del src, dst
        return P.GigabytesPerSecond(n * 4 / (st.median_us * 1e-6) / 1e9)

    # -- this package's measurements ---------------------------------------

    def time_stats(self, operation: Callable[[], Any], warmup: int = 25, timed: int = 100, flush: bool = True,
                   graph: bool = False) -> LatencyStats:
        """Microseconds per call, one event pair per sample on the current
        stream. `graph=True` captures the operation once in a HIP graph and
        times its replays, as a decode runtime issues it: without the ~2 us a
        host-side dispatch adds to every eager launch."""
        run = operation
        if graph:
            for _ in range(3):
                operation()
            cur = torch.cuda.current_stream()
            side = torch.cuda.Stream()
            side.wait_stream(cur)
            with torch.cuda.stream(side):
                operation()
            cur.wait_stream(side)
            torch.cuda.synchronize(self.device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                operation()
            torch.cuda.synchronize(self.device)
            run = g.replay
        for _ in range(warmup):
            run()
        torch.cuda.synchronize(self.device)
        out = []
        for _ in range(timed):
            if flush:
                self.flush()
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            run()
            e.record()
            e.synchronize()
            out.append(s.elapsed_time(e) * 1000.0)
        return latency_stats(out)

    def time_cold_rotation(self, operations, warmup: int = 25, timed: int = 100) -> LatencyStats:
        """Microseconds per launch of `operations`, each reading its own copy
        of the data (together several times L2 + Infinity Cache, so every
        launch reads HBM), captured back to back in one HIP graph: each sample
        is one replay divided by the launches in it. This is how a decode
        step issues its products; a graph of a single launch instead carries
        a per-replay cost of ~10 us on this GPU, and an eager launch ~2 us of
        host dispatch."""
        ops = list(operations)

        def seq():
            for op in ops:
                op()

        seq()
        cur = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            seq()
        cur.wait_stream(side)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            seq()
        torch.cuda.synchronize(self.device)
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize(self.device)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(timed + 1)]
        ev[0].record()
        for i in range(timed):
            g.replay()
            ev[i + 1].record()
        ev[-1].synchronize()
        out = latency_stats([ev[i].elapsed_time(ev[i + 1]) * 1000.0 / len(ops) for i in range(timed)])
        del g
        return out

    def measure_stream_read_bandwidth(self, nbytes: int = 1 << 30, copies: int = 4) -> float:
        """GB/s of the library's streaming-read probe over `copies` buffers of
        `nbytes` (each over 4x L2 + Infinity Cache), one launch per buffer in
        one graph: the read-only traffic of a weight pass."""
        dev = f"cuda:{self.device}"
        bufs = [torch.zeros(nbytes, dtype=torch.uint8, device=dev) for _ in range(copies)]
        sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
        lib = nat.lib()

        def probe(b):
            return lambda: nat.check(lib.se12_read_probe(nat.ptr(b), b.numel(), nat.ptr(sink), sink.numel(),
                                                         nat.stream_ptr()))

        st = self.time_cold_rotation([probe(b) for b in bufs], warmup=3, timed=10)
        del bufs
        return nbytes / (st.median_us * 1e-6) / 1e9

    def measure_graph_launch_us(self, launches: int = 64) -> float:
        """Microseconds per node of a HIP graph of `launches` dependent
        one-element kernels: the fixed cost a launch adds to a decode step."""
        t = torch.zeros(1, dtype=torch.float32, device=f"cuda:{self.device}")

        def chain():
            for _ in range(launches):
                t.add_(1.0)

        st = self.time_stats(chain, warmup=5, timed=20, flush=False, graph=True)
        return st.median_us / launches

    def measure_copy_traffic_gbps(self, nbytes: int = 1 << 30) -> float:
        """GB/s of HBM traffic of a device-to-device copy of `nbytes`, read
        and write both counted: the copy's physical rate, for the roofline
        (the port's measure_peak_copy_bandwidth counts the bytes once)."""
        n = nbytes // 4
        src = torch.empty(n, dtype=torch.float32, device=f"cuda:{self.device}")
        dst = torch.empty_like(src)
        st = self.time_stats(lambda: dst.copy_(src), warmup=5, timed=20, flush=False)
        return 2 * n * 4 / (st.median_us * 1e-6) / 1e9


def median(values) -> float:
    return float(_st.median(values))
