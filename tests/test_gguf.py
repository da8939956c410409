"""GGUF loader (combsengine_amd.gguf) on CPU: the reference's synthetic-file
round trip, metadata types, rejections, RoPE row de-permutation against an
independent restatement of llama.cpp's forward permutation, phi3 fused-row
slicing, and the loader feeding try_quant_linear (GPU)."""
import struct

import numpy as np
import pytest

import oracle as O
from combsengine_amd import QuantFormat, ModelError, quantize, try_quant_linear
from combsengine_amd.gguf import GgufSource, map_tensor_name, rope_depermute_src_rows
from gguf_writer import (T_ARRAY, T_BOOL, T_F32, T_F64, T_I16, T_I32, T_I64, T_I8, T_STRING, T_U16, T_U32,
                         T_U64, T_U8, write_gguf)


def _q8_block(d_half_bits: int, vals) -> bytes:
    return struct.pack("<H", d_half_bits) + bytes(v & 0xFF for v in vals)


def _llama_kv(hidden=64, heads=1, kv_heads=1, layers=1, ffn=128, arch="llama"):
    return [("general.architecture", T_STRING, arch),
            (f"{arch}.embedding_length", T_U32, hidden),
            (f"{arch}.attention.head_count", T_U32, heads),
            (f"{arch}.attention.head_count_kv", T_U32, kv_heads),
            (f"{arch}.block_count", T_U32, layers),
            (f"{arch}.context_length", T_U32, 128),
            (f"{arch}.feed_forward_length", T_U32, ffn)]


def test_reference_round_trip_fixture(tmp_path):
    """The file of combs-formats/tests/gguf.rs:10-89 (tiny llama, Q8_0
    token_embd d = 0.5, q = +-2; F32 output_norm), checked as in
    gguf.rs:91-125: metadata, names, tied head, Q8_0 values +-1.0."""
    kv = _llama_kv() + [("tokenizer.ggml.eos_token_id", T_U32, 7),
                        ("tokenizer.ggml.tokens", T_ARRAY, (T_STRING, ["<s>", "a", "b", "c", "d", "e", "f", "</s>"])),
                        ("tokenizer.ggml.merges", T_ARRAY, (T_STRING, []))]
    q8 = b"".join(_q8_block(0x3800, [2 if j % 2 == 0 else -2 for j in range(32)]) for _ in range(16))
    norm = struct.pack("<64f", *([1.0] * 64))
    path = tmp_path / "tiny.gguf"
    write_gguf(path, kv, [("token_embd.weight", [64, 8], 8, q8), ("output_norm.weight", [64], 0, norm)],
               pad_between=False)
    src = GgufSource.load(path)
    md = src.metadata
    assert (md.architecture, md.hidden_size, md.num_hidden_layers, md.num_attention_heads) == ("llama", 64, 1, 1)
    assert md.max_position_embeddings == 128 and md.eos_token_ids == [7] and md.vocab_size == 8
    assert md.tie_word_embeddings
    names = src.tensor_names()
    assert "model.embed_tokens.weight" in names and "model.norm.weight" in names
    qt = src.open_tensor_quant("model.embed_tokens.weight")
    assert qt.format == QuantFormat.Q8_0 and qt.shape == [8, 64]
    vals = O.dequant(O.Q8_0, bytes(qt.data), 512)
    assert vals[0] == 1.0 and vals[1] == -1.0 and np.all(np.abs(vals) == 1.0)
    assert src.open_tensor_quant("model.norm.weight") is None  # F32: not a packed tensor
    assert src.open_tensor_quant("model.layers.0.mlp.up_proj.weight") is None  # absent


def test_metadata_value_types(tmp_path):
    kv = _llama_kv() + [("t.u8", T_U8, 250), ("t.i8", T_I8, -5), ("t.u16", T_U16, 65000), ("t.i16", T_I16, -300),
                        ("t.i32", T_I32, -70000), ("t.f32", T_F32, 1.5), ("t.bool", T_BOOL, 1),
                        ("t.u64", T_U64, 1 << 40), ("t.i64", T_I64, -(1 << 40)), ("t.f64", T_F64, 0.25),
                        ("t.arr", T_ARRAY, (T_I32, [1, -2, 3])), ("general.alignment", T_U32, 64)]
    path = tmp_path / "types.gguf"
    write_gguf(path, kv, [("token_embd.weight", [32, 1], 8, _q8_block(0x3C00, range(32)))], align=64)
    src = GgufSource.load(path)
    assert src.kv["t.u8"] == 250 and src.kv["t.i8"] == -5 and src.kv["t.u16"] == 65000
    assert src.kv["t.i16"] == -300 and src.kv["t.i32"] == -70000 and src.kv["t.f32"] == 1.5
    assert src.kv["t.bool"] is True and src.kv["t.u64"] == 1 << 40 and src.kv["t.i64"] == -(1 << 40)
    assert src.kv["t.f64"] == 0.25 and src.kv["t.arr"] == [1, -2, 3]
    assert src.data_start % 64 == 0
    qt = src.open_tensor_quant("model.embed_tokens.weight")
    assert bytes(qt.data) == _q8_block(0x3C00, range(32))


def test_rejections(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + b"\0" * 64)
    with pytest.raises(ModelError, match="magic"):
        GgufSource.load(p)
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 4, 0, 0))
    with pytest.raises(ModelError, match="version"):
        GgufSource.load(p)
    write_gguf(p, _llama_kv() + [("split.count", T_U16, 3), ("split.no", T_U16, 1)], [])
    with pytest.raises(ModelError, match="shard 2 of 3"):
        GgufSource.load(p)
    write_gguf(p, [("general.architecture", T_STRING, "llama")], [])
    with pytest.raises(ModelError, match="embedding_length"):
        GgufSource.load(p)


def test_name_map():
    """gguf.rs:645-682."""
    assert map_tensor_name("blk.3.attn_q.weight", "llama") == "model.layers.3.self_attn.q_proj.weight"
    assert map_tensor_name("blk.0.ffn_down.weight", "qwen2") == "model.layers.0.mlp.down_proj.weight"
    assert map_tensor_name("blk.1.ffn_norm.weight", "llama") == "model.layers.1.post_attention_layernorm.weight"
    assert map_tensor_name("blk.1.ffn_norm.weight", "gemma3") == "model.layers.1.pre_feedforward_layernorm.weight"
    assert map_tensor_name("output.weight", "llama") == "lm_head.weight"
    assert map_tensor_name("rope_freqs.weight", "llama") is None
    assert map_tensor_name("blk.0.attn_qkv.weight", "phi3") is None


def _llamacpp_permute(w: np.ndarray, n_head: int) -> np.ndarray:
    """llama.cpp convert_hf_to_gguf's forward permutation of q/k rows (HF
    rotate-half -> ggml interleaved pairs), restated from its published
    reshape: rows (n_head, 2, d/2) -> (n_head, d/2, 2)."""
    rows = w.shape[0]
    return w.reshape(n_head, 2, rows // n_head // 2, *w.shape[1:]).swapaxes(1, 2).reshape(w.shape)


def test_depermute_map_inverts_llamacpp_permute():
    for rows, heads in ((64, 1), (64, 4), (128, 8), (96, 3)):
        hf = np.arange(rows)
        stored = _llamacpp_permute(hf, heads)
        assert np.array_equal(stored[rope_depermute_src_rows(rows, heads)], hf)


@pytest.mark.parametrize("fmt", [QuantFormat.Q8_0, QuantFormat.Q4K, QuantFormat.Q6K])
def test_rope_rows_depermuted(tmp_path, fmt):
    """llama attn_q (4 heads) and attn_k (2 kv heads) stored in llama.cpp's
    permuted row order come back in HF order; qwen2 rows are served verbatim."""
    heads, kv_heads, d, k = 4, 2, 16, 256
    rng = np.random.default_rng(3)
    q_hf = rng.normal(0, 1, (heads * d, k)).astype(np.float32)
    k_hf = rng.normal(0, 1, (kv_heads * d, k)).astype(np.float32)
    qb = np.frombuffer(quantize(fmt, q_hf), np.uint8).reshape(heads * d, -1)
    kb = np.frombuffer(quantize(fmt, k_hf), np.uint8).reshape(kv_heads * d, -1)
    q_st, k_st = _llamacpp_permute(qb, heads), _llamacpp_permute(kb, kv_heads)
    for arch, expect_q, expect_k in (("llama", qb, kb), ("mistral", qb, kb), ("qwen2", q_st, k_st)):
        path = tmp_path / f"{arch}.gguf"
        write_gguf(path, _llama_kv(hidden=heads * d, heads=heads, kv_heads=kv_heads, arch=arch),
                   [("blk.0.attn_q.weight", [k, heads * d], int(fmt), q_st.tobytes()),
                    ("blk.0.attn_k.weight", [k, kv_heads * d], int(fmt), k_st.tobytes())])
        src = GgufSource.load(path)
        q = src.open_tensor_quant("model.layers.0.self_attn.q_proj.weight")
        kk = src.open_tensor_quant("model.layers.0.self_attn.k_proj.weight")
        assert q.shape == [heads * d, k] and kk.shape == [kv_heads * d, k]
        assert bytes(q.data) == expect_q.tobytes(), arch
        assert bytes(kk.data) == expect_k.tobytes(), arch


def test_phi3_fused_row_slices(tmp_path):
    """phi3 attn_qkv = [q|k|v] rows, ffn_up = [gate|up] rows (gguf.rs:1034-1059)."""
    heads, kv_heads, hd, ffn, k = 4, 2, 8, 48, 256
    qkv_rows = (heads + 2 * kv_heads) * hd
    qkv = np.arange(qkv_rows * k // 32 * 34, dtype=np.uint32).astype(np.uint8).reshape(qkv_rows, -1)
    up = (np.arange(2 * ffn * k // 32 * 34, dtype=np.uint32) * 7).astype(np.uint8).reshape(2 * ffn, -1)
    kv = _llama_kv(hidden=heads * hd, heads=heads, kv_heads=kv_heads, ffn=ffn, arch="phi3")
    path = tmp_path / "phi3.gguf"
    write_gguf(path, kv, [("blk.0.attn_qkv.weight", [k, qkv_rows], 8, qkv.tobytes()),
                          ("blk.0.ffn_up.weight", [k, 2 * ffn], 8, up.tobytes())])
    src = GgufSource.load(path)
    q_rows, kv_rows = heads * hd, kv_heads * hd
    for name, data, lo, n in (("self_attn.q_proj", qkv, 0, q_rows), ("self_attn.k_proj", qkv, q_rows, kv_rows),
                              ("self_attn.v_proj", qkv, q_rows + kv_rows, kv_rows),
                              ("mlp.gate_proj", up, 0, ffn), ("mlp.up_proj", up, ffn, ffn)):
        qt = src.open_tensor_quant(f"model.layers.0.{name}.weight")
        assert qt.shape == [n, k], name
        assert bytes(qt.data) == data[lo:lo + n].tobytes(), name
    assert "model.layers.0.self_attn.v_proj.weight" in src.tensor_names()


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", [QuantFormat.Q4K, QuantFormat.Q8_0])
def test_gguf_feeds_quant_linear(cuda, tmp_path, fmt):
    """A llama GGUF's attn_q (permuted on disk) through try_quant_linear:
    the op computes x . W_hf^T against the oracle on the de-permuted rows."""
    import torch
    heads, d, k = 4, 32, 512
    rng = np.random.default_rng(9)
    w_hf = rng.normal(0, 0.02, (heads * d, k)).astype(np.float32)
    packed = np.frombuffer(quantize(fmt, w_hf), np.uint8).reshape(heads * d, -1)
    path = tmp_path / "m.gguf"
    write_gguf(path, _llama_kv(hidden=heads * d, heads=heads, kv_heads=heads),
               [("blk.0.attn_q.weight", [k, heads * d], int(fmt), _llamacpp_permute(packed, heads).tobytes())])
    op = try_quant_linear(GgufSource.load(path), "model.layers.0.self_attn.q_proj.weight")
    assert op is not None and op.dims() == [heads * d, k]
    x = rng.normal(0, 1, (1, 3, k)).astype(np.float16)
    y = op.forward(torch.from_numpy(x).cuda()).float().cpu().numpy().reshape(3, heads * d)
    wd = O.dequant(int(fmt), packed.tobytes(), heads * d * k).reshape(heads * d, k)
    O.assert_close(y, O.ref_matmul(x.reshape(3, k).astype(np.float32), wd), 1e-3, "gguf q_proj")
