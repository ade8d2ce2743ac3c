"""CPU: token files (llmt.tokens, the counterpart of python/tokenize_input.py
and python/decode_tokens.py).  The file layout is [int32 n][n int32 ids]
(src/train.cu:202-205): checked byte for byte against struct packing, and
the tokenizer path runs on a word-level tokenizer built here (no download)."""
import struct

import numpy as np
import pytest

from llmt import tokens


def test_layout_is_header_then_ids(tmp_path):
    ids = [0, 7, 151935, 42, 2**31 - 1]
    p = tmp_path / "t.bin"
    assert tokens.write_token_file(p, ids) == 5
    want = struct.pack("<i", 5) + b"".join(struct.pack("<i", i) for i in ids)
    assert p.read_bytes() == want
    assert tokens.read_token_file(p).tolist() == ids


def test_empty_and_bad_files(tmp_path):
    p = tmp_path / "e.bin"
    tokens.write_token_file(p, [])
    assert tokens.read_token_file(p).size == 0
    bad = tmp_path / "b.bin"
    np.array([4, 1, 2], dtype="<i4").tofile(bad)  # header says 4, holds 2
    with pytest.raises(ValueError):
        tokens.read_token_file(bad)
    with pytest.raises(ValueError):
        tokens.write_token_file(tmp_path / "x.bin", [2**31])


def _word_tokenizer(path):
    tk = pytest.importorskip("tokenizers")
    vocab = {"<unk>": 0, "the": 1, "cat": 2, "sat": 3, "on": 4, "mat": 5}
    t = tk.Tokenizer(tk.models.WordLevel(vocab, unk_token="<unk>"))
    t.pre_tokenizer = tk.pre_tokenizers.Whitespace()
    t.decoder = tk.decoders.WordPiece()
    t.save(str(path))
    return path


def test_cli_prompt_train_and_decode(tmp_path, capsys):
    tj = _word_tokenizer(tmp_path / "tokenizer.json")
    out = tmp_path / "data" / "input_tokens.bin"
    assert tokens.main(["--tokenizer", str(tj), "--out", str(out), "the cat sat"]) == 0
    assert tokens.read_token_file(out).tolist() == [1, 2, 3]
    corpus = tmp_path / "corpus.txt"
    corpus.write_text("the cat sat on the mat\nthe dog")
    tr = tmp_path / "data" / "train_tokens.bin"
    assert tokens.main(["--tokenizer", str(tj), "--train", str(corpus), "--out", str(tr)]) == 0
    assert tokens.read_token_file(tr).tolist() == [1, 2, 3, 4, 1, 5, 1, 0]
    capsys.readouterr()
    assert tokens.main(["--tokenizer", str(tj), "--decode", "1", "2", "3"]) == 0
    assert capsys.readouterr().out.strip() == "the cat sat"
