"""CPU: adapter files <-> PEFT adapters (llmt.peft, the counterpart of
python/save_lora.py).

The key names and shapes are pinned against a random-init transformers
Qwen3ForCausalLM: every PEFT key must name one of its attention projections,
with lora_A [r, in_features] and lora_B [out_features, r] of that module's
weight.  Round trips through each output format must reproduce the adapter
files byte for byte, and the adapter config's lora_alpha / r must be the
step's LoRA scale (2.0, src/kernels/lora.cu:181-202)."""
import json

import numpy as np
import pytest

from llmt import peft
from oracle import lora_step as ref

TINY = peft.AdapterDims(n_layers=2, hidden=64, n_heads=4, n_kv_heads=2, head_dim=16, rank=16,
                        alpha=32.0)


def _write_random(d, step, dims, seed=0):
    rng = np.random.default_rng(seed)
    for layer in range(dims.n_layers):
        for proj, (d_out, d_in) in dims.shapes().items():
            for mat, shape in (("A", (dims.rank, d_in)), ("B", (d_out, dims.rank))):
                rng.standard_normal(shape).astype("<f4").tofile(
                    peft.bin_path(d, step, layer, proj, mat))


def _files(d):
    return {p.name: p.read_bytes() for p in sorted(d.iterdir())}


@pytest.mark.parametrize("form", ["dir", "file.safetensors", "state.pt"])
def test_round_trip_is_byte_exact(tmp_path, form):
    src, dst = tmp_path / "src", tmp_path / "dst"
    src.mkdir()
    _write_random(src, 7, TINY)
    out = tmp_path / form
    peft.to_peft(src, 7, out, TINY)
    peft.from_peft(out, dst, 7, TINY)
    assert _files(src) == _files(dst)
    assert len(_files(dst)) == TINY.n_layers * 8


def test_keys_and_shapes_match_hf_qwen3(tmp_path):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen3Config(vocab_size=32, hidden_size=TINY.hidden, intermediate_size=96,
                                   num_hidden_layers=TINY.n_layers,
                                   num_attention_heads=TINY.n_heads,
                                   num_key_value_heads=TINY.n_kv_heads, head_dim=TINY.head_dim,
                                   tie_word_embeddings=True)
    sd = transformers.Qwen3ForCausalLM(cfg).state_dict()
    _write_random(tmp_path, 0, TINY)
    state = peft.read_adapters(tmp_path, 0, TINY)
    assert len(state) == TINY.n_layers * 8
    for key, arr in state.items():
        assert key.startswith("base_model.model.")
        module, mat = key[len("base_model.model."):].rsplit(".lora_", 1)
        w = sd[module + ".weight"]
        out_f, in_f = w.shape
        if mat == "A.weight":
            assert arr.shape == (TINY.rank, in_f)
        else:
            assert mat == "B.weight"
            assert arr.shape == (out_f, TINY.rank)


def test_values_land_in_the_named_projection(tmp_path):
    # layer 1's wo B file becomes layer 1's o_proj lora_B, row-major [d_out, r]
    _write_random(tmp_path, 3, TINY, seed=5)
    raw = np.fromfile(peft.bin_path(tmp_path, 3, 1, "wo", "B"), dtype="<f4")
    state = peft.read_adapters(tmp_path, 3, TINY)
    b = state["base_model.model.model.layers.1.self_attn.o_proj.lora_B.weight"]
    assert b.shape == (TINY.hidden, TINY.rank)
    assert np.array_equal(b.ravel(), raw)
    assert b[2, 5] == raw[2 * TINY.rank + 5]


def test_config_scale_is_the_step_scale(tmp_path):
    _write_random(tmp_path, 0, TINY)
    peft.to_peft(tmp_path, 0, tmp_path / "hf", TINY)
    cfg = json.loads((tmp_path / "hf" / "adapter_config.json").read_text())
    assert cfg["lora_alpha"] / cfg["r"] == ref.Dims().lora_scale == 2.0
    assert sorted(cfg["target_modules"]) == ["k_proj", "o_proj", "q_proj", "v_proj"]


def test_missing_and_misshapen_inputs_raise(tmp_path):
    _write_random(tmp_path, 0, TINY)
    state = peft.read_adapters(tmp_path, 0, TINY)
    bad = dict(state)
    del bad["base_model.model.model.layers.0.self_attn.k_proj.lora_A.weight"]
    with pytest.raises(KeyError):
        peft.write_adapters(bad, tmp_path / "x", 0, TINY)
    bad = dict(state)
    bad["base_model.model.model.layers.1.self_attn.q_proj.lora_B.weight"] = np.zeros((3, 16))
    with pytest.raises(ValueError):
        peft.write_adapters(bad, tmp_path / "y", 0, TINY)
    # a truncated adapter file
    p = peft.bin_path(tmp_path, 0, 0, "wv", "B")
    np.zeros(5, dtype="<f4").tofile(p)
    with pytest.raises(ValueError):
        peft.read_adapters(tmp_path, 0, TINY)


def test_cli_list(tmp_path, capsys):
    _write_random(tmp_path, 2, TINY)
    # the CLI lists the Qwen3-1.7B adapters by file presence (as
    # save_lora.py --list): layers 0-1 are present here, the rest missing
    assert peft.main(["--list", "--step", "2", "--weights-dir", str(tmp_path)]) == 0
    out = capsys.readouterr().out
    assert "layer  0  wq  A=16x2048" in out
    assert "layer 27  wo  MISSING" in out
