"""Expert weight formats and safetensors ingest for the MoE layer.

Mirrors the subset of nano_ktrans/kernels/weight_loader.py that the MoE
expert path reads:

* ``GPTQLinearWeight`` (weight_loader.py:25-69): ``qweight`` int32
  [out, in*bits/32] with value j of word w = input column (32/bits)*w + j,
  stored as q + 2^(bits-1); ``scales`` [out, groups]; symmetric only.
* ``ExpertWeightLoader`` (weight_loader.py:72-421): safetensors key index,
  dense per-expert loads with the packed ``gate_up`` split (355-392) and the
  GPTQ on-disk transform (278-325: ``qweight`` transposed from [in/8, out],
  scales [groups, out] or [out, groups], sequential ``g_idx`` only).
  Extension: ``group_size = -1`` (one group per row) for int8 per-channel
  checkpoints, which the reference's loader cannot express.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass
from glob import glob
from typing import Dict, List, Optional

import torch


@dataclass
class GPTQLinearWeight:
    qweight: torch.Tensor
    scales: torch.Tensor
    zero_points: Optional[torch.Tensor]
    group_size: int
    bits: int
    sym: bool
    linear_prefix: str

    @property
    def input_dim(self) -> int:
        return int(self.qweight.shape[1]) * self.values_per_word

    @property
    def output_dim(self) -> int:
        return int(self.qweight.shape[0])

    @property
    def num_groups(self) -> int:
        return int(self.scales.shape[1])

    @property
    def values_per_word(self) -> int:
        return 32 // self.bits

    def unpack_qvalues(self) -> torch.Tensor:
        shifts = torch.arange(self.values_per_word, dtype=torch.int32, device=self.qweight.device) * self.bits
        packed = self.qweight.to(dtype=torch.int32).contiguous()
        unpacked = ((packed.unsqueeze(-1) >> shifts) & ((1 << self.bits) - 1)).to(dtype=torch.float32)
        return unpacked.reshape(self.output_dim, self.qweight.shape[1] * self.values_per_word)

    def dequantize(self) -> torch.Tensor:
        q = self.unpack_qvalues()
        zero = float(1 << (self.bits - 1))
        g = self.num_groups
        gs = self.input_dim // g
        s = self.scales.to(torch.float32).repeat_interleave(gs, dim=1)
        return (q - zero) * s


class ExpertWeightLoader:
    """Read MoE expert weights from a directory of ``*.safetensors`` files."""

    def __init__(self, weight_path: str):
        from safetensors import safe_open  # noqa: F401  (fail early if absent)

        self.weight_path = weight_path
        self._key_to_file: Dict[str, str] = {}
        self._quantize_config: Dict[str, object] = {}
        self._handles: Dict[str, object] = {}
        if not weight_path:
            return
        files = sorted(glob(os.path.join(weight_path, "*.safetensors")))
        if not files:
            raise FileNotFoundError(f"No .safetensors files found in {weight_path}")
        from safetensors import safe_open

        for f in files:
            with safe_open(f, "pt", "cpu") as sf:
                for key in sf.keys():
                    self._key_to_file[key] = f
        self._quantize_config = self._load_quantize_config()

    def _load_quantize_config(self) -> Dict[str, object]:
        for filename in ("quantize_config.json", "config.json"):
            path = os.path.join(self.weight_path, filename)
            if not os.path.exists(path):
                continue
            try:
                with open(path, "r", encoding="utf-8") as handle:
                    payload = json.load(handle)
            except (OSError, json.JSONDecodeError):
                continue
            if filename == "quantize_config.json":
                return payload
            quant = payload.get("quantization_config")
            if isinstance(quant, dict):
                return quant
        return {}

    def has_key(self, key: str) -> bool:
        return key in self._key_to_file

    def load_tensor(self, key: str) -> torch.Tensor:
        """One tensor by its checkpoint key (contiguous, on the CPU)."""
        return self._load_tensor(key)

    def _load_tensor(self, key: str) -> torch.Tensor:
        file_path = self._key_to_file.get(key)
        if file_path is None:
            raise KeyError(f"Weight key '{key}' not found in safetensors files.")
        handle = self._handles.get(file_path)
        if handle is None:
            from safetensors import safe_open

            handle = safe_open(file_path, "pt", "cpu").__enter__()
            self._handles[file_path] = handle
        return handle.get_tensor(key).contiguous()

    def load_expert(
        self,
        layer_idx: int,
        expert_idx: int,
        key_template: str = "model.layers.{layer}.block_sparse_moe.experts.{expert}.{proj}.weight",
        proj_name_map: Optional[Dict[str, str]] = None,
    ) -> Dict[str, torch.Tensor]:
        """Dense gate/up/down of one expert; a packed ``gate_up`` is split (gate rows first)."""
        proj_map = proj_name_map or {"gate": "w1", "up": "w3", "down": "w2"}
        result: Dict[str, torch.Tensor] = {}
        for proj_name, w_name in proj_map.items():
            tensor = self._load_tensor(key_template.format(layer=layer_idx, expert=expert_idx, proj=w_name))
            if proj_name == "gate_up":
                gate, up = tensor.chunk(2, dim=0)
                result["gate"] = gate.contiguous()
                result["up"] = up.contiguous()
            else:
                result[proj_name] = tensor
        return result

    def load_gptq_linear(
        self,
        linear_prefix: str,
        *,
        bits: Optional[int] = None,
        group_size: Optional[int] = None,
        sym: Optional[bool] = None,
    ) -> GPTQLinearWeight:
        bits = int(bits or self._quantize_config.get("bits", 4))
        gs_cfg = group_size if group_size is not None else self._quantize_config.get("group_size", 128)
        group_size = int(gs_cfg)
        sym = bool(self._quantize_config.get("sym", True) if sym is None else sym)
        if not sym:
            raise NotImplementedError("Asymmetric GPTQ weights are not supported.")
        qweight = self._load_tensor(f"{linear_prefix}.qweight").transpose(0, 1).to(torch.int32).contiguous()
        scales_raw = self._load_tensor(f"{linear_prefix}.scales")
        output_dim = qweight.shape[0]
        input_dim = qweight.shape[1] * (32 // bits)
        if group_size == -1:
            group_size = input_dim
        num_groups = (input_dim + group_size - 1) // group_size
        g_idx_key = f"{linear_prefix}.g_idx"
        if g_idx_key in self._key_to_file:
            g_idx = self._load_tensor(g_idx_key).to(dtype=torch.long)
            expected = torch.arange(input_dim, dtype=torch.long) // group_size
            if g_idx.numel() < input_dim or not torch.equal(g_idx[:input_dim], expected):
                raise NotImplementedError("Only sequential GPTQ grouping is supported.")
        if tuple(scales_raw.shape) == (output_dim, num_groups):
            scales = scales_raw.to(torch.float32).contiguous()
        elif tuple(scales_raw.shape) == (num_groups, output_dim):
            scales = scales_raw.transpose(0, 1).to(torch.float32).contiguous()
        else:
            raise ValueError(
                f"Unsupported GPTQ scales shape {tuple(scales_raw.shape)} for "
                f"out={output_dim}, groups={num_groups}")
        return GPTQLinearWeight(qweight, scales, None, group_size, bits, sym, linear_prefix)

    def load_gptq_expert_linear(
        self,
        *,
        layer_idx: int,
        expert_idx: int,
        proj_name: str,
        key_template: str = "model.layers.{layer}.mlp.experts.{expert}.{proj}.weight",
        proj_name_map: Optional[Dict[str, str]] = None,
    ) -> GPTQLinearWeight:
        proj_map = proj_name_map or {"gate": "gate_proj", "up": "up_proj", "down": "down_proj"}
        key = key_template.format(layer=layer_idx, expert=expert_idx, proj=proj_map[proj_name])
        prefix = key[: -len(".weight")] if key.endswith(".weight") else key
        return self.load_gptq_linear(prefix)

    def is_gptq_expert(self, layer_idx: int, expert_idx: int, key_template: str,
                       proj_name_map: Dict[str, str]) -> bool:
        first = list(proj_name_map.values())[0]
        key = key_template.format(layer=layer_idx, expert=expert_idx, proj=first)
        prefix = key[: -len(".weight")] if key.endswith(".weight") else key
        return f"{prefix}.qweight" in self._key_to_file

    def layer_keys(self) -> List[str]:
        return sorted(self._key_to_file)
