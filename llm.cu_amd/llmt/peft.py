"""LoRA adapter files <-> HuggingFace PEFT adapters.

Counterpart of python/save_lora.py (list :65-78, --to-hf :81-98, --from-hf
:101-116): the adapter files are the ones llmt_lora_save / llm_train write,
<dir>/lora_step{N}_layer{L}_{wq|wk|wv|wo}_{A|B}.bin (src/train.cu:146-170),
raw little-endian fp32, A [rank, d_in] and B [d_out, rank] row-major.  PEFT
keys are base_model.model.model.layers.{L}.self_attn.{q|k|v|o}_proj.lora_{A|B}.weight
with the same shapes (save_lora.py:88-91).

Output formats: a directory (PEFT's adapter_model.safetensors plus an
adapter_config.json with r = rank and lora_alpha = alpha, so PEFT's scaling
lora_alpha / r is the step's 2.0), a single .safetensors file, or a torch
state dict (.pt, the reference's format).  Inputs are read only with loaders
that execute nothing from the file (safetensors; torch.load with
weights_only=True).

  python -m llmt.peft --list --step 100 [--weights-dir weights]
  python -m llmt.peft --to-hf --step 100 --out weights/lora_hf_step100
  python -m llmt.peft --from-hf --adapter path/to/adapter --step 0
"""

import argparse
import json
import os
from dataclasses import dataclass

import numpy as np

PROJ_HF = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj",
           "wo": "self_attn.o_proj"}


@dataclass(frozen=True)
class AdapterDims:
    """Adapter shapes of the model (Qwen3-1.7B by default)."""
    n_layers: int = 28
    hidden: int = 2048
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    rank: int = 16
    alpha: float = 32.0

    def shapes(self):
        """(d_out, d_in) of each adapted projection, in file order."""
        q, kv = self.n_heads * self.head_dim, self.n_kv_heads * self.head_dim
        return {"wq": (q, self.hidden), "wk": (kv, self.hidden), "wv": (kv, self.hidden),
                "wo": (self.hidden, q)}


def bin_path(weights_dir, step: int, layer: int, proj: str, mat: str) -> str:
    return os.path.join(str(weights_dir), f"lora_step{step}_layer{layer}_{proj}_{mat}.bin")


def peft_key(layer: int, proj: str, mat: str) -> str:
    return f"base_model.model.model.layers.{layer}.{PROJ_HF[proj]}.lora_{mat}.weight"


def _read_f32(path: str, shape) -> np.ndarray:
    n = int(np.prod(shape))
    data = np.fromfile(path, dtype="<f4")
    if data.size != n:
        raise ValueError(f"{path}: {data.size} floats, expected {n} for {tuple(shape)}")
    return data.reshape(shape)


def read_adapters(weights_dir, step: int, dims: AdapterDims = AdapterDims()) -> dict:
    """Every adapter file of one step as PEFT-keyed fp32 arrays."""
    out = {}
    for layer in range(dims.n_layers):
        for proj, (d_out, d_in) in dims.shapes().items():
            out[peft_key(layer, proj, "A")] = _read_f32(
                bin_path(weights_dir, step, layer, proj, "A"), (dims.rank, d_in))
            out[peft_key(layer, proj, "B")] = _read_f32(
                bin_path(weights_dir, step, layer, proj, "B"), (d_out, dims.rank))
    return out


def write_adapters(state: dict, weights_dir, step: int, dims: AdapterDims = AdapterDims()):
    """PEFT-keyed arrays (any float dtype) -> the adapter files of one step."""
    os.makedirs(str(weights_dir), exist_ok=True)
    for layer in range(dims.n_layers):
        for proj, (d_out, d_in) in dims.shapes().items():
            for mat, shape in (("A", (dims.rank, d_in)), ("B", (d_out, dims.rank))):
                key = peft_key(layer, proj, mat)
                if key not in state:
                    raise KeyError(f"adapter has no {key}")
                arr = np.asarray(state[key], dtype=np.float32)
                if arr.shape != shape:
                    raise ValueError(f"{key}: shape {arr.shape}, expected {shape}")
                arr.astype("<f4").tofile(bin_path(weights_dir, step, layer, proj, mat))


def adapter_config(dims: AdapterDims, base_model: str = "Qwen/Qwen3-1.7B") -> dict:
    return {"peft_type": "LORA", "task_type": "CAUSAL_LM", "base_model_name_or_path": base_model,
            "r": dims.rank, "lora_alpha": dims.alpha, "lora_dropout": 0.0, "bias": "none",
            "target_modules": ["q_proj", "k_proj", "v_proj", "o_proj"], "fan_in_fan_out": False}


def to_peft(weights_dir, step: int, out, dims: AdapterDims = AdapterDims()) -> str:
    """Adapter files -> a PEFT adapter directory, a .safetensors file or a
    .pt state dict (by the form of `out`); returns the file written."""
    state = read_adapters(weights_dir, step, dims)
    out = str(out)
    if out.endswith(".pt") or out.endswith(".bin"):
        import torch
        torch.save({k: torch.from_numpy(v) for k, v in state.items()}, out)
        return out
    from safetensors.numpy import save_file
    if out.endswith(".safetensors"):
        save_file(state, out)
        return out
    os.makedirs(out, exist_ok=True)
    path = os.path.join(out, "adapter_model.safetensors")
    save_file(state, path)
    with open(os.path.join(out, "adapter_config.json"), "w") as f:
        json.dump(adapter_config(dims), f, indent=2)
    return path


def load_peft(src) -> dict:
    """PEFT-keyed arrays from an adapter directory, a .safetensors file or a
    torch state dict (weights only)."""
    src = str(src)
    if os.path.isdir(src):
        src = os.path.join(src, "adapter_model.safetensors")
    if src.endswith(".safetensors"):
        from safetensors.numpy import load_file
        return load_file(src)
    import torch
    state = torch.load(src, map_location="cpu", weights_only=True)
    return {k: v.float().numpy() for k, v in state.items()}


def from_peft(src, weights_dir, step: int, dims: AdapterDims = AdapterDims()) -> None:
    write_adapters(load_peft(src), weights_dir, step, dims)


def list_adapters(weights_dir, step: int, dims: AdapterDims = AdapterDims()) -> int:
    """Print every adapter of one step (present or missing); returns the
    parameter count of those present."""
    total = 0
    for layer in range(dims.n_layers):
        for proj, (d_out, d_in) in dims.shapes().items():
            pa = bin_path(weights_dir, step, layer, proj, "A")
            pb = bin_path(weights_dir, step, layer, proj, "B")
            if os.path.exists(pa) and os.path.exists(pb):
                total += dims.rank * (d_in + d_out)
                print(f"  layer {layer:2d}  {proj}  A={dims.rank}x{d_in}  B={d_out}x{dims.rank}")
            else:
                print(f"  layer {layer:2d}  {proj}  MISSING")
    print(f"\nTotal LoRA parameters: {total:,}  ({total * 4 / 1e6:.1f} MB)")
    return total


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--step", type=int, default=0)
    ap.add_argument("--list", action="store_true")
    ap.add_argument("--to-hf", action="store_true")
    ap.add_argument("--from-hf", action="store_true")
    ap.add_argument("--adapter", default="")
    ap.add_argument("--out", default="weights/lora_hf")
    ap.add_argument("--weights-dir", default="weights")
    a = ap.parse_args(argv)
    if a.list:
        list_adapters(a.weights_dir, a.step)
    elif a.to_hf:
        print(f"Saved PEFT adapter to {to_peft(a.weights_dir, a.step, a.out)}")
    elif a.from_hf:
        if not a.adapter:
            ap.error("--adapter required")
        from_peft(a.adapter, a.weights_dir, a.step)
        print(f"Exported {AdapterDims().n_layers * 8} adapter files to {a.weights_dir}/")
    else:
        ap.print_help()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
