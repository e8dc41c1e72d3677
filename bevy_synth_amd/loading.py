"""Safetensors loading of the TRELLIS2 sparse decoder onto the device: the
Python twin of include/sparse_decoder_loading.hpp, after
crates/burn_trellis/src/runtime_model/sparse_decoder_loading.rs.

* ``SafeTensors``         : the file (8-byte little-endian header length, JSON
                            header, byte buffer); ``load_tensor_f32`` decodes
                            f32 / f16 / bf16 payloads (:231-310), other dtypes
                            refused; ``load_vector`` (:210-229).
* ``load_sparse_conv``    : weight [Cout, KD, KH, KW, Cin_g] + bias (:93-200).
* ``load_linear``, ``load_linear_dynamic``: weight [Cout, Cin] + bias (:1-91).
* ``load_decoder_stage``  : one stage of SparseStructuredLatentDecoder::
                            from_safetensors (sparse_decoder_runtime_impl.rs
                            :94-190): ConvNeXt blocks ``blocks.{s}.{b}.{conv,
                            norm, mlp.0, mlp.2}``, then (all but the last stage)
                            the C2S upsample ``blocks.{s}.{N}.{norm1, to_subdiv,
                            conv1, conv2}``.

Checks, their order and the error messages are the reference's (raised as
``LoadError``), so a caller's handling carries over.  Layers land on the
device in the compute dtype: bf16 and f16 through the library's
round-to-nearest-even conversion (sc_convert), f32 as is; biases and the
to_subdiv weights stay f32, f16-rounded in f16 mode (the reference's
weight_fp16 / bias_fp16 copies, sparse_decoder.rs:780-793).
"""
from __future__ import annotations

import json
import struct
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from . import decoder as D
from .flex_gmm import SparseSubmConvConfig, convert


class LoadError(ValueError):
    """A refused tensor or layer (the reference's Err(String))."""


_DTYPES = {"F32": np.dtype("<f4"), "F16": np.dtype("<f2"), "BF16": np.dtype("<u2")}


class SafeTensors:
    """An opened safetensors file (read whole into host memory)."""

    def __init__(self, header: Dict[str, dict], data: bytes):
        self._t = header
        self._data = data

    @classmethod
    def open(cls, path: str) -> "SafeTensors":
        try:
            with open(path, "rb") as f:
                blob = f.read()
        except OSError:
            raise LoadError(f"cannot open safetensors file '{path}'") from None
        if len(blob) < 8:
            raise LoadError(f"safetensors file '{path}' is shorter than its 8-byte header length")
        (n,) = struct.unpack("<Q", blob[:8])
        if n > len(blob) - 8:
            raise LoadError(f"safetensors header length {n} exceeds the file")
        try:
            header = json.loads(blob[8:8 + n].decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise LoadError(f"malformed safetensors header: {e}") from None
        if not isinstance(header, dict):
            raise LoadError("header is not a JSON object")
        header.pop("__metadata__", None)
        data = blob[8 + n:]
        for key, t in header.items():
            b, e = t["data_offsets"]
            if e > len(data) or b > e:
                raise LoadError(f"tensor '{key}' data_offsets exceed the buffer")
        return cls(header, data)

    def contains(self, key: str) -> bool:
        return key in self._t

    def load_tensor_f32(self, key: str) -> Tuple[Tuple[int, ...], np.ndarray]:
        """(shape, values decoded to f32), load_tensor_f32 :231-266."""
        t = self._t.get(key)
        if t is None:
            raise LoadError(f"missing tensor '{key}' in safetensors")
        b, e = t["data_offsets"]
        raw = self._data[b:e]
        dt = t["dtype"]
        if dt == "F32":
            if len(raw) % 4:
                raise LoadError(f"invalid f32 tensor payload byte length {len(raw)}; must be divisible by 4")
            out = np.frombuffer(raw, _DTYPES[dt]).astype(np.float32)
        elif dt in ("F16", "BF16"):
            if len(raw) % 2:
                raise LoadError(f"invalid {dt.lower()} tensor payload byte length {len(raw)}; "
                                "must be divisible by 2")
            h = np.frombuffer(raw, _DTYPES[dt])
            out = (h.astype(np.float32) if dt == "F16"
                   else (h.astype(np.uint32) << 16).view(np.float32))
        else:
            raise LoadError(f"tensor '{key}' has unsupported dtype {dt}; expected f32/f16/bf16")
        shape = tuple(int(d) for d in t["shape"])
        expected = int(np.prod(shape, dtype=np.int64)) if shape else 1
        if out.size != expected:
            raise LoadError(f"tensor '{key}' element count mismatch: expected {expected}, got {out.size}")
        return shape, out.reshape(shape)

    def load_vector(self, key: str, expected_len: int) -> np.ndarray:
        """load_vector :210-229."""
        shape, v = self.load_tensor_f32(key)
        if len(shape) != 1:
            raise LoadError(f"tensor '{key}' expected rank=1, got rank={len(shape)}")
        if expected_len > 0 and shape[0] != expected_len:
            raise LoadError(f"tensor '{key}' expected len={expected_len}, got len={shape[0]}")
        return v


def _upload(v: np.ndarray, dtype: torch.dtype, device) -> torch.Tensor:
    """Host f32 values -> device tensor of the compute dtype (RNE on the device)."""
    t = torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)).to(device)
    return t if dtype == torch.float32 else convert(t, dtype)


def _upload_f32(v: np.ndarray, dtype: torch.dtype, device) -> torch.Tensor:
    """An f32 operand (bias, to_subdiv weight): f16-rounded in f16 mode."""
    t = torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)).to(device)
    return convert(convert(t, torch.float16), torch.float32) if dtype == torch.float16 else t


def _check_dtype(dtype: torch.dtype) -> None:
    if dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise LoadError("compute dtype must be f32, bf16 or f16")


def load_sparse_conv(st: SafeTensors, weight_key: str, bias_key: str, expected_in: int, expected_out: int,
                     dtype: torch.dtype = torch.bfloat16, device=None) -> D.ConvLayer:
    """load_sparse_conv, sparse_decoder_loading.rs:93-200: groups =
    expected_in / Cin_g (Cin_g when expected_in is 0)."""
    _check_dtype(dtype)
    ws, w = st.load_tensor_f32(weight_key)
    if len(ws) != 5:
        raise LoadError(f"tensor '{weight_key}' expected rank=5, got rank={len(ws)}")
    out_channels, kd, kh, kw, in_pg = ws
    if kd == 0 or kh == 0 or kw == 0:
        raise LoadError(f"tensor '{weight_key}' has invalid kernel dims ({kd},{kh},{kw})")
    if in_pg == 0:
        raise LoadError(f"tensor '{weight_key}' has invalid in_channels_per_group=0")
    if expected_out > 0 and out_channels != expected_out:
        raise LoadError(f"tensor '{weight_key}' expected out_channels={expected_out}, got {out_channels}")
    in_channels = expected_in if expected_in > 0 else in_pg
    if in_channels < in_pg or in_channels % in_pg != 0:
        raise LoadError(f"tensor '{weight_key}' expected_in={in_channels} is incompatible with "
                        f"in_per_group={in_pg}")
    groups = in_channels // in_pg
    if groups == 0 or out_channels % groups != 0:
        raise LoadError(f"tensor '{weight_key}' has incompatible grouped channels (groups={groups}, "
                        f"out_channels={out_channels})")
    bs, b = st.load_tensor_f32(bias_key)
    if len(bs) != 1 or bs[0] != out_channels:
        raise LoadError(f"tensor '{bias_key}' expected shape=[{out_channels}]")
    cfg = SparseSubmConvConfig(in_channels, out_channels, kd, kh, kw, in_channels_per_group=in_pg,
                               out_channels_per_group=out_channels // groups, groups=groups)
    dev = torch.device("cuda") if device is None else torch.device(device)
    return D.ConvLayer(cfg, _upload(w.reshape(out_channels, kd * kh * kw, in_pg), dtype, dev),
                       _upload_f32(b, dtype, dev))


def _load_linear(st: SafeTensors, weight_key: str, bias_key: str, expected_in: int, expected_out: int,
                 dtype: torch.dtype, device, f32_weight: bool = False) -> D.LinearLayer:
    _check_dtype(dtype)
    ws, w = st.load_tensor_f32(weight_key)
    if len(ws) != 2:
        raise LoadError(f"tensor '{weight_key}' expected rank=2, got rank={len(ws)}")
    out_channels, in_channels = ws
    if expected_in > 0 and in_channels != expected_in:
        raise LoadError(f"tensor '{weight_key}' expected in_channels={expected_in}, got {in_channels}")
    if expected_out > 0 and out_channels != expected_out:
        raise LoadError(f"tensor '{weight_key}' expected out_channels={expected_out}, got {out_channels}")
    bs, b = st.load_tensor_f32(bias_key)
    if len(bs) != 1 or bs[0] != out_channels:
        raise LoadError(f"tensor '{bias_key}' expected shape=[{out_channels}]")
    dev = torch.device("cuda") if device is None else torch.device(device)
    wt = _upload_f32(w, dtype, dev) if f32_weight else _upload(w, dtype, dev)
    return D.LinearLayer(wt, _upload_f32(b, dtype, dev))


def load_linear(st: SafeTensors, weight_key: str, bias_key: str, expected_in: int, expected_out: int,
                dtype: torch.dtype = torch.bfloat16, device=None) -> D.LinearLayer:
    """load_linear, sparse_decoder_loading.rs:1-48."""
    return _load_linear(st, weight_key, bias_key, expected_in, expected_out, dtype, device)


def load_linear_dynamic(st: SafeTensors, weight_key: str, bias_key: str, expected_in: int,
                        dtype: torch.dtype = torch.bfloat16, device=None) -> D.LinearLayer:
    """load_linear_dynamic, sparse_decoder_loading.rs:50-91 (output width from
    the file: the ConvNeXt MLP's hidden width)."""
    return _load_linear(st, weight_key, bias_key, expected_in, 0, dtype, device)


def load_decoder_stage(st: SafeTensors, stage_idx: int, num_blocks: int, stage_channels: int,
                       next_channels: int, pred_subdiv: bool = True, dtype: torch.dtype = torch.bfloat16,
                       device=None) -> D.TrellisDecoderStage:
    """Stage ``stage_idx`` of the decoder (sparse_decoder_runtime_impl.rs
    :94-190): ``num_blocks`` ConvNeXt blocks at ``stage_channels``
    (model_channels[s]) and, when ``next_channels`` > 0 (model_channels[s+1];
    0 for the last stage), the upsample to ``next_channels`` whose to_subdiv
    head (Linear Cin -> 8, f32) is read when ``pred_subdiv`` is set.  Keys,
    expected shapes, load order and messages are the reference's; the first
    failure is raised."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    blocks: List[D.ConvNeXtBlock] = []
    for b in range(num_blocks):
        pre = f"blocks.{stage_idx}.{b}"
        conv = load_sparse_conv(st, f"{pre}.conv.weight", f"{pre}.conv.bias", stage_channels, stage_channels,
                                dtype, dev)
        nw = st.load_vector(f"{pre}.norm.weight", stage_channels)
        nb = st.load_vector(f"{pre}.norm.bias", stage_channels)
        m0 = load_linear_dynamic(st, f"{pre}.mlp.0.weight", f"{pre}.mlp.0.bias", stage_channels, dtype, dev)
        m2 = load_linear_dynamic(st, f"{pre}.mlp.2.weight", f"{pre}.mlp.2.bias", 0, dtype, dev)
        blocks.append(D.ConvNeXtBlock(conv, torch.from_numpy(nw).to(dev), torch.from_numpy(nb).to(dev), m0, m2))
    up = None
    if next_channels > 0:
        pre = f"blocks.{stage_idx}.{num_blocks}"
        ts = (_load_linear(st, f"{pre}.to_subdiv.weight", f"{pre}.to_subdiv.bias", stage_channels, 8, dtype, dev,
                           f32_weight=True) if pred_subdiv else None)
        n1w = st.load_vector(f"{pre}.norm1.weight", stage_channels)
        n1b = st.load_vector(f"{pre}.norm1.bias", stage_channels)
        c1 = load_sparse_conv(st, f"{pre}.conv1.weight", f"{pre}.conv1.bias", stage_channels, 8 * next_channels,
                              dtype, dev)
        c2 = load_sparse_conv(st, f"{pre}.conv2.weight", f"{pre}.conv2.bias", next_channels, next_channels,
                              dtype, dev)
        up = D.C2SUpsampleBlock(stage_channels, next_channels, torch.from_numpy(n1w).to(dev),
                                torch.from_numpy(n1b).to(dev), c1, c2,
                                to_subdiv_weight=None if ts is None else ts.weight,
                                to_subdiv_bias=None if ts is None else ts.bias,
                                compute_fp16=dtype == torch.float16)
    return D.TrellisDecoderStage(blocks, up)
