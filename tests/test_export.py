"""CPU: a Hugging Face safetensors checkpoint -> the reference's weight files
(llmt.export, the counterpart of python/export_weights.py:12-29 and
scripts/run.sh:19).  A random-init transformers Qwen3ForCausalLM saved with
save_pretrained is exported; every file must hold its parameter as raw fp32
row-major bytes, the file set must be what llmt_load_weights_dir reads, and
a tied head must come out as a copy of the embedding."""
import numpy as np
import pytest

from llmt import export

transformers = pytest.importorskip("transformers")
torch = pytest.importorskip("torch")


def _tiny(tied, dtype):
    torch.manual_seed(3)
    cfg = transformers.Qwen3Config(vocab_size=48, hidden_size=32, intermediate_size=64,
                                   num_hidden_layers=2, num_attention_heads=2,
                                   num_key_value_heads=1, head_dim=16, tie_word_embeddings=tied)
    return transformers.Qwen3ForCausalLM(cfg).to(dtype)


def _loader_names(n_layers):
    """The files llmt_load_weights_dir opens (src/train.cu:56-89)."""
    names = {"model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"}
    for l in range(n_layers):
        for m in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                  "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj", "input_layernorm",
                  "post_attention_layernorm", "self_attn.q_norm", "self_attn.k_norm"):
            names.add(f"model.layers.{l}.{m}.weight")
    return names


@pytest.mark.parametrize("tied", [True, False])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_export_tiny_qwen3(tmp_path, tied, dtype):
    model = _tiny(tied, getattr(torch, dtype))
    model.save_pretrained(tmp_path / "ckpt", safe_serialization=True)
    names = export.export_checkpoint(tmp_path / "ckpt", tmp_path / "w")
    assert set(names) == _loader_names(2)
    sd = model.state_dict()
    for name in names:
        got = np.fromfile(tmp_path / "w" / f"{name}.bin", dtype="<f4")
        want = sd[name].to(torch.float32).numpy()
        assert got.size == want.size
        assert np.array_equal(got, want.ravel()), name
    emb = (tmp_path / "w" / "model.embed_tokens.weight.bin").read_bytes()
    head = (tmp_path / "w" / "lm_head.weight.bin").read_bytes()
    assert (emb == head) == tied


def test_export_needs_safetensors(tmp_path):
    with pytest.raises(FileNotFoundError):
        export.export_checkpoint(tmp_path, tmp_path / "w")
