"""The Python layer's checks of caller-supplied tensors, without a GPU:
host tensors, wrong dtypes, shapes or layouts and short streams are refused
before any pointer would cross into the library; the attention rule of the
runtime refuses transformers' eager attention on a HIP device."""

from __future__ import annotations

import pytest
import torch

from oracle import se12_codec as o
from se12_amd import hip, runtime
from se12_amd.format import Se12DeviceTensor, validate_device_streams

DEV = torch.device("cuda", 0)   # a device name only: nothing is allocated on it


def test_require_refuses_host_misshapen_and_strided_tensors():
    t = torch.zeros((2, 8), dtype=torch.float32)
    with pytest.raises(ValueError, match="is on cpu"):
        hip._require(t, "out", torch.float32, (2, 8), DEV)
    assert hip._require(t, "out", torch.float32, (2, 8), t.device) is t
    with pytest.raises(ValueError, match="float32"):
        hip._require(t.to(torch.bfloat16), "out", torch.float32, (2, 8), t.device)
    with pytest.raises(ValueError):
        hip._require(t, "out", torch.float32, (2, 9), t.device)
    with pytest.raises(ValueError, match="not contiguous"):
        hip._require(torch.zeros((8, 2)).t(), "out", torch.float32, (2, 8), t.device)
    with pytest.raises(ValueError, match="torch tensor"):
        hip._require(None, "out", torch.float32, (2, 8), DEV)


def _host_streams_as_device_tensor(rows=32, cols=512):
    bits = o.normal_bf16(rows, cols, seed=0, std=0.02)
    enc = o.encode(bits.reshape(-1), rows, cols)
    return Se12DeviceTensor(sm=torch.from_numpy(enc["sm"]), ec=torch.from_numpy(enc["ec"]),
                            esc=torch.from_numpy(enc["esc"].reshape(-1)), codebook=torch.from_numpy(enc["codebook"]),
                            fallback_bitmap=torch.from_numpy(enc["fallback_bitmap"]),
                            fallback_raw=torch.from_numpy(enc["fallback_raw"]), rows=rows, cols=cols,
                            codebook_host=tuple(int(c) for c in enc["codebook"]))


def test_device_streams_must_live_on_a_gpu():
    dt = _host_streams_as_device_tensor()
    with pytest.raises(ValueError, match="device tensors"):
        validate_device_streams(dt)
    with pytest.raises(ValueError, match="device tensors"):
        hip._as_device_tensor(dt)


def test_attention_rule_on_a_hip_device():
    assert runtime.resolve_attention(None, torch.device("cpu")) is None
    assert runtime.resolve_attention("eager", torch.device("cpu")) == "eager"
    assert runtime.resolve_attention("sdpa", DEV) == "sdpa"
    with pytest.raises(ValueError, match="faulted"):
        runtime.resolve_attention("eager", DEV)
    pytest.importorskip("transformers")
    assert runtime.resolve_attention(None, DEV) == runtime.CONTIGUOUS_EAGER
