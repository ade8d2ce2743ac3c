"""Token files for llm_train: [int32 n][n x int32 ids], little-endian.

Counterpart of python/tokenize_input.py:14-37 (a prompt -> data/input_tokens.bin,
--train <text file> -> data/train_tokens.bin) and python/decode_tokens.py:9-17
(ids -> text, special tokens skipped), with the tokenizer read from a local
directory or tokenizer.json (the reference fetches Qwen/Qwen3-1.7B's; there is
no download here).  The file format is the one src/train.cu:202-205 reads.

  python -m llmt.tokens --tokenizer path/to/Qwen3-1.7B "your prompt here"
  python -m llmt.tokens --tokenizer path/to/Qwen3-1.7B --train corpus.txt
  python -m llmt.tokens --tokenizer path/to/Qwen3-1.7B --decode 9707 11 1879
"""

import argparse
import os

import numpy as np


def write_token_file(path, ids) -> int:
    """Write ids as a token file; returns the count."""
    a = np.asarray(ids, dtype=np.int64)
    if a.ndim != 1 or (a.size and (a.min() < -2**31 or a.max() >= 2**31)):
        raise ValueError("token ids must be a flat sequence of int32 values")
    d = os.path.dirname(str(path))
    if d:
        os.makedirs(d, exist_ok=True)
    with open(str(path), "wb") as f:
        np.array([a.size], dtype="<i4").tofile(f)
        a.astype("<i4").tofile(f)
    return int(a.size)


def read_token_file(path) -> np.ndarray:
    raw = np.fromfile(str(path), dtype="<i4")
    if raw.size < 1 or raw[0] < 0 or raw[0] != raw.size - 1:
        raise ValueError(f"{path}: header says {raw[0] if raw.size else 'nothing'}, "
                         f"file holds {max(raw.size - 1, 0)} ids")
    return raw[1:].astype(np.int32)


def load_tokenizer(path):
    """A local tokenizer: a directory transformers' AutoTokenizer can open
    (local_files_only), or a tokenizer.json for the tokenizers library."""
    path = str(path)
    if os.path.isdir(path):
        from transformers import AutoTokenizer
        return AutoTokenizer.from_pretrained(path, local_files_only=True)
    from tokenizers import Tokenizer
    return Tokenizer.from_file(path)


def encode(tok, text: str) -> list:
    ids = tok.encode(text)
    return list(ids.ids) if hasattr(ids, "ids") else list(ids)


def decode(tok, ids) -> str:
    return tok.decode([int(i) for i in ids], skip_special_tokens=True)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--tokenizer", required=True, help="tokenizer directory or tokenizer.json")
    ap.add_argument("--train", metavar="TEXT_FILE", help="tokenize a corpus")
    ap.add_argument("--decode", nargs="+", type=int, metavar="ID", help="ids -> text")
    ap.add_argument("--out", help="output file (default data/train_tokens.bin or "
                                  "data/input_tokens.bin)")
    ap.add_argument("prompt", nargs="?")
    a = ap.parse_args(argv)
    tok = load_tokenizer(a.tokenizer)
    if a.decode:
        print(decode(tok, a.decode))
        return 0
    if a.train:
        with open(a.train) as f:
            ids = encode(tok, f.read())
        out = a.out or "data/train_tokens.bin"
        print(f"Wrote {write_token_file(out, ids)} tokens to {out}")
        return 0
    if a.prompt is None:
        ap.error("a prompt, --train or --decode is required")
    ids = encode(tok, a.prompt)
    out = a.out or "data/input_tokens.bin"
    print(f"Wrote {write_token_file(out, ids)} tokens to {out}")
    print(f"Token IDs: {ids}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
