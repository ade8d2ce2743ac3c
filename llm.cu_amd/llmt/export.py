"""A local Hugging Face checkpoint -> the reference's weight files.

Counterpart of python/export_weights.py:12-29 (every parameter as
<out>/<hf_param_name>.bin, raw little-endian fp32, row-major [out, in], no
header) and of scripts/run.sh:19 (lm_head.weight.bin as a copy of the
embedding when the checkpoint ties them).  The checkpoint is read from its
*.safetensors files (one or sharded, any float dtype) one tensor at a time,
with nothing fetched and nothing executed from the files; llmt_load_weights_dir
reads the result.

  python -m llmt.export --checkpoint path/to/Qwen3-1.7B --out weights
"""

import argparse
import glob
import os
import shutil


def export_checkpoint(checkpoint, out_dir, verbose: bool = False) -> list:
    """Write every tensor of the checkpoint as <out_dir>/<name>.bin fp32;
    returns the names written (lm_head.weight included)."""
    import torch
    from safetensors import safe_open
    files = sorted(glob.glob(os.path.join(str(checkpoint), "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no *.safetensors in {checkpoint}")
    os.makedirs(str(out_dir), exist_ok=True)
    names = []
    for path in files:
        with safe_open(path, framework="pt") as f:
            for name in f.keys():
                t = f.get_tensor(name).to(torch.float32).contiguous()
                t.numpy().astype("<f4").tofile(os.path.join(str(out_dir), name + ".bin"))
                names.append(name)
                if verbose:
                    print(f"    {name}: {list(t.shape)}")
    if "lm_head.weight" not in names:
        if "model.embed_tokens.weight" not in names:
            raise KeyError("checkpoint has neither lm_head.weight nor model.embed_tokens.weight")
        shutil.copyfile(os.path.join(str(out_dir), "model.embed_tokens.weight.bin"),
                        os.path.join(str(out_dir), "lm_head.weight.bin"))
        names.append("lm_head.weight")
    return names


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--checkpoint", required=True, help="directory with *.safetensors")
    ap.add_argument("--out", default="weights")
    a = ap.parse_args(argv)
    names = export_checkpoint(a.checkpoint, a.out, verbose=True)
    print(f"\nExported {len(names)} tensors to {a.out}/")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
