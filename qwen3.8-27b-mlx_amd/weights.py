"""Reader for the Gated-DeltaNet layers' weights in the reference's checkpoint format
(safetensors shards + config.json), into the layouts the kernels take.

Follows the reference's loader (paths relative to the reference tree):
  cpp/src/model.cpp:272-340  Config::from_json (text_config keys, quantization block)
  cpp/src/model.cpp:733-754  load_model: every *.safetensors shard of the directory, names
                             with "model.language_model." or "model." stripped
  cpp/src/model.cpp:149-183  deltanet(): conv1d.weight (C, 1, K) -> (K, C), A_log and
                             dt_bias to fp32, the five projections, the gated norm
  cpp/src/model.cpp:80-104   gated_rmsnorm (gamma as stored, fp32: not zero-centred) and
                             linear (4-bit: weight (N, K/8) uint32 + scales + biases (N, K/64))
Tensors are read with safetensors (no code in the file is executed).
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional

from .gdn import CONV_TAPS, HEAD_DIM, QuantLinear

_PREFIXES = ("model.language_model.", "model.")


def _strip(name: str) -> str:
    for p in _PREFIXES:
        if name.startswith(p):
            return name[len(p):]
    return name


@dataclass
class DeltaNetConfig:
    """The text_config fields the DeltaNet layers use (model.cpp:272-340; defaults are the
    reference's Config defaults)."""
    hidden_size: int = 5120
    num_hidden_layers: int = 64
    layer_types: List[str] = field(default_factory=list)
    linear_num_key_heads: int = 16
    linear_num_value_heads: int = 48
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    linear_conv_kernel_dim: int = 4
    rms_norm_eps: float = 1e-6
    quantized: bool = False
    group_size: int = 64
    bits: int = 4
    quantized_modules: List[str] = field(default_factory=list)

    @classmethod
    def from_json(cls, path: str) -> "DeltaNetConfig":
        raw = json.load(open(path))
        t = raw.get("text_config")
        if not isinstance(t, dict):
            raise ValueError("config.json has no text_config")
        c = cls()
        for k in ("hidden_size", "num_hidden_layers", "linear_num_key_heads", "linear_num_value_heads",
                  "linear_key_head_dim", "linear_value_head_dim", "linear_conv_kernel_dim"):
            setattr(c, k, int(t.get(k, getattr(c, k))))
        c.rms_norm_eps = float(t.get("rms_norm_eps", c.rms_norm_eps))
        lt = t.get("layer_types")
        if not isinstance(lt, list) or not lt:
            raise ValueError("config.json has no text_config.layer_types")
        if len(lt) != c.num_hidden_layers:
            raise ValueError(f"layer_types has {len(lt)} entries but num_hidden_layers is "
                             f"{c.num_hidden_layers}")
        c.layer_types = [str(x) for x in lt]
        q = raw.get("quantization")
        if isinstance(q, dict):
            c.quantized = True
            c.group_size = int(q.get("group_size", 64))
            c.bits = int(q.get("bits", 4))
            c.quantized_modules = [str(m) for m in q.get("quantized_modules", [])]
        return c

    def is_quantized(self, path: str) -> bool:
        """Config::is_quantized (model.cpp:266-270)."""
        mods = set(self.quantized_modules)
        return path in mods or ("model.language_model." + path) in mods or ("model." + path) in mods


@dataclass
class PlainLinear:
    """A projection stored in bf16 (not quantized): weight (N, K)."""
    weight: object

    @property
    def n(self) -> int:
        return self.weight.shape[0]


@dataclass
class DeltaNetLayerWeights:
    """One Gated-DeltaNet layer's parameters in the kernels' layouts (device tensors)."""
    conv_weight: object        # (K, C) bf16: w[j, c] = conv1d.weight[c, 0, j]
    A_log: object              # (Hv,) fp32
    dt_bias: object            # (Hv,) fp32
    norm_gamma: object         # (Dv,) fp32, as stored (the gated norm is not zero-centred)
    in_proj_qkv: object        # QuantLinear (4-bit) or PlainLinear
    in_proj_z: object
    in_proj_a: object
    in_proj_b: object
    out_proj: object


class Checkpoint:
    """A checkpoint directory: config.json and *.safetensors shards (model.cpp:733-754)."""

    def __init__(self, model_dir: str):
        from safetensors import safe_open
        self.dir = model_dir
        self.config = DeltaNetConfig.from_json(os.path.join(model_dir, "config.json"))
        shards = sorted(f for f in os.listdir(model_dir) if f.endswith(".safetensors"))
        if not shards:
            raise FileNotFoundError(f"no .safetensors files in {model_dir}")
        self._where: Dict[str, tuple] = {}
        for f in shards:
            path = os.path.join(model_dir, f)
            with safe_open(path, framework="pt", device="cpu") as st:
                for name in st.keys():
                    self._where[_strip(name)] = (path, name)

    def names(self) -> List[str]:
        return sorted(self._where)

    def tensor(self, name: str):
        """The named tensor (prefixes stripped) on the CPU, as stored."""
        from safetensors import safe_open
        if name not in self._where:
            raise KeyError(f"checkpoint is missing tensor '{name}'")
        path, full = self._where[name]
        with safe_open(path, framework="pt", device="cpu") as st:
            return st.get_tensor(full)

    def _take(self, name: str, shape):
        t = self.tensor(name)
        if shape is not None and tuple(t.shape) != tuple(shape):
            raise ValueError(f"tensor '{name}' has shape {tuple(t.shape)}, expected {tuple(shape)}")
        return t

    def _linear(self, path: str, out_f: int, in_f: int, device):
        import torch
        c = self.config
        if c.quantized and c.is_quantized(path):
            if c.bits != 4 or c.group_size != 64:
                raise ValueError(f"{path}: {c.bits}-bit group {c.group_size} weights; the kernels take 4-bit group 64")
            w = self._take(path + ".weight", None)
            if w.shape[0] != out_f or w.shape[1] * 32 // c.bits != in_f:
                raise ValueError(f"tensor '{path}.weight' has shape {tuple(w.shape)}, expected "
                                 f"({out_f}, {in_f * c.bits // 32})")
            s = self._take(path + ".scales", (out_f, in_f // c.group_size))
            b = self._take(path + ".biases", (out_f, in_f // c.group_size))
            return QuantLinear(w.view(torch.int32).to(device), s.to(torch.bfloat16).to(device),
                               b.to(torch.bfloat16).to(device))
        w = self._take(path + ".weight", (out_f, in_f))
        return PlainLinear(w.to(torch.bfloat16).to(device))

    def deltanet_layer(self, i: int, device="cuda") -> DeltaNetLayerWeights:
        """deltanet() for layers.{i}.linear_attn (model.cpp:149-183, 236)."""
        import torch
        c = self.config
        if c.layer_types[i] != "linear_attention":
            raise ValueError(f"layer {i} is {c.layer_types[i]}, not linear_attention")
        path = f"layers.{i}.linear_attn"
        nk, nv = c.linear_num_key_heads, c.linear_num_value_heads
        dk, dv, K, h = c.linear_key_head_dim, c.linear_value_head_dim, c.linear_conv_kernel_dim, c.hidden_size
        # the kernels implement 4 conv taps, 128-wide heads and an integer number of v-heads
        # per k-head (include/gdn.h): anything else would load and then be misread
        if K != CONV_TAPS:
            raise ValueError(f"linear_conv_kernel_dim = {K}; the kernels take {CONV_TAPS} taps")
        if dk != HEAD_DIM or dv != HEAD_DIM:
            raise ValueError(f"linear key/value head dims = {dk}/{dv}; the kernels take {HEAD_DIM}")
        if nk < 1 or nv < 1 or nv % nk != 0:
            raise ValueError(f"linear_num_value_heads = {nv} is not a multiple of linear_num_key_heads = {nk}")
        qkv_dim, z_dim = 2 * nk * dk + nv * dv, nv * dv
        conv = self._take(path + ".conv1d.weight", (qkv_dim, 1, K))
        return DeltaNetLayerWeights(
            conv_weight=conv[:, 0, :].t().contiguous().to(torch.bfloat16).to(device),
            A_log=self._take(path + ".A_log", (nv,)).float().to(device),
            dt_bias=self._take(path + ".dt_bias", (nv,)).float().to(device),
            norm_gamma=self._take(path + ".norm.weight", (dv,)).float().to(device),
            in_proj_qkv=self._linear(path + ".in_proj_qkv", qkv_dim, h, device),
            in_proj_z=self._linear(path + ".in_proj_z", z_dim, h, device),
            in_proj_a=self._linear(path + ".in_proj_a", nv, h, device),
            in_proj_b=self._linear(path + ".in_proj_b", nv, h, device),
            out_proj=self._linear(path + ".out_proj", h, z_dim, device),
        )

    def deltanet_layers(self, device="cuda") -> Dict[int, DeltaNetLayerWeights]:
        return {i: self.deltanet_layer(i, device) for i, t in enumerate(self.config.layer_types)
                if t == "linear_attention"}
