"""GGUF file reader feeding the quantized linear layer: the parts of
combs_formats::GgufSource (engine/core/combs-formats/src/gguf.rs) that the
quantized path consumes.

- `GgufSource.load(path)` (gguf.rs:213-319): memory-maps the file; parses the
  header (magic, version 2..3, tensor and metadata counts), the metadata
  key/values (gguf.rs:117-196), the tensor infos (name, ggml dims, ggml type,
  offset) and the data start (aligned to `general.alignment`, default 32);
  rejects split-file shards; builds the model metadata the path needs
  (gguf.rs:331-398) and marks tied embeddings when `output.weight` is absent.
- `open_tensor_quant(hf_name)` (gguf.rs:1233-1289): resolves the HF tensor
  name to its ggml tensor (gguf.rs:645-682, phi3 fused projections
  gguf.rs:1034-1080), returns the packed block bytes as a `QuantTensor` with
  the HF shape [n_out, k] (ggml dims reversed), sliced to a fused projection's
  row range and, for llama / mistral `attn_q` / `attn_k`, with its rows
  de-permuted from llama.cpp's interleaved RoPE layout back to rotate-half
  (gguf.rs:1000-1031).  None for tensor types the kernels do not take.

The tensor bytes are served from the mmap (zero-copy) unless rows are
reordered.  Tokenizer synthesis, sampler defaults and the dense tensor
reader of the reference are callers of this path, not part of it.
"""
import mmap
import os
import struct
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np

from .qlinear import ModelError, QuantFormat, QuantTensor, tensor_byte_size

GGUF_MAGIC = 0x46554747  # "GGUF"

# metadata value types (gguf.rs:117-129)
META_U8, META_I8, META_U16, META_I16, META_U32, META_I32, META_F32 = 0, 1, 2, 3, 4, 5, 6
META_BOOL, META_STRING, META_ARRAY, META_U64, META_I64, META_F64 = 7, 8, 9, 10, 11, 12

_SCALAR = {META_U8: "<B", META_I8: "<b", META_U16: "<H", META_I16: "<h", META_U32: "<I", META_I32: "<i",
           META_F32: "<f", META_BOOL: "<B", META_U64: "<Q", META_I64: "<q", META_F64: "<d"}

# ggml tensor types served by the quantized path (gguf.rs:1237-1245), plus
# Q4_1 (3) and Q5_1 (7), which the reference leaves to its dense path
_GGML_QUANT = {2: QuantFormat.Q4_0, 3: QuantFormat.Q4_1, 6: QuantFormat.Q5_0, 7: QuantFormat.Q5_1, 8: QuantFormat.Q8_0,
               12: QuantFormat.Q4K, 13: QuantFormat.Q5K, 14: QuantFormat.Q6K}


class _Cursor:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.buf):
            raise ModelError("gguf: unexpected end of file")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return bytes(b)

    def unpack(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.unpack("<Q")
        return self.take(n).decode("utf-8")


def _read_value(c: _Cursor, ty: int):
    """read_meta_value (gguf.rs:131-196): scalars, strings, arrays of them."""
    if ty in _SCALAR:
        v = c.unpack(_SCALAR[ty])
        return bool(v) if ty == META_BOOL else v
    if ty == META_STRING:
        return c.string()
    if ty == META_ARRAY:
        elem, n = c.unpack("<I"), c.unpack("<Q")
        if elem not in _SCALAR and elem != META_STRING:
            raise ModelError(f"gguf: unsupported metadata array element type {elem}")
        return [_read_value(c, elem) for _ in range(n)]
    raise ModelError(f"gguf: unsupported metadata type {ty}")


@dataclass
class TensorInfo:
    name: str
    dims: List[int]      # ggml order: innermost (k) first
    ggml_type: int
    offset: int          # from the data start


@dataclass
class ModelMetadata:
    """The fields of ModelMetadata (gguf.rs:331-398) this path uses."""
    architecture: str
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    max_position_embeddings: int
    vocab_size: int
    eos_token_ids: List[int]
    bos_token_id: Optional[int]
    tie_word_embeddings: bool = False


def map_tensor_name(ggml: str, arch: str) -> Optional[str]:
    """ggml tensor name -> HF name (gguf.rs:645-682)."""
    top = {"token_embd.weight": "model.embed_tokens.weight", "output.weight": "lm_head.weight",
           "output_norm.weight": "model.norm.weight"}
    if ggml in top:
        return top[ggml]
    if not ggml.startswith("blk."):
        return None
    layer, _, rest = ggml[4:].partition(".")
    if not rest:
        return None
    gemma = arch in ("gemma3", "gemma3_text")
    table = {
        "attn_norm.weight": "input_layernorm.weight",
        "attn_q_norm.weight": "self_attn.q_norm.weight",
        "attn_k_norm.weight": "self_attn.k_norm.weight",
        "attn_q.weight": "self_attn.q_proj.weight",
        "attn_k.weight": "self_attn.k_proj.weight",
        "attn_v.weight": "self_attn.v_proj.weight",
        "attn_output.weight": "self_attn.o_proj.weight",
        "attn_q.bias": "self_attn.q_proj.bias",
        "attn_k.bias": "self_attn.k_proj.bias",
        "attn_v.bias": "self_attn.v_proj.bias",
        "attn_output.bias": "self_attn.o_proj.bias",
        "ffn_gate.weight": "mlp.gate_proj.weight",
        "ffn_up.weight": "mlp.up_proj.weight",
        "ffn_down.weight": "mlp.down_proj.weight",
    }
    if gemma:
        table.update({"ffn_norm.weight": "pre_feedforward_layernorm.weight",
                      "post_attention_norm.weight": "post_attention_layernorm.weight",
                      "post_ffw_norm.weight": "post_feedforward_layernorm.weight"})
    else:
        table["ffn_norm.weight"] = "post_attention_layernorm.weight"
    hf = table.get(rest)
    return f"model.layers.{layer}.{hf}" if hf else None


def rope_depermute_src_rows(rows: int, n_head: int) -> np.ndarray:
    """For each HF (rotate-half) row, the ggml (interleaved-pairs) row it is
    read from, per head of d = rows / n_head rows: hf[j] = ggml[2j] for
    j < d/2, else ggml[2(j - d/2) + 1] (gguf.rs:1000-1020)."""
    d = rows // n_head
    half = d // 2
    j = np.arange(d)
    within = np.where(j < half, 2 * j, 2 * (j - half) + 1)
    return (np.arange(n_head)[:, None] * d + within[None, :]).reshape(-1)


class GgufSource:
    """A parsed, memory-mapped GGUF file (GgufSource, gguf.rs:211-319)."""

    def __init__(self, path, mm, kv, tensors, data_start, metadata):
        self.path = path
        self._mm = mm
        self.kv: Dict[str, object] = kv
        self.tensors: Dict[str, TensorInfo] = tensors
        self.data_start = data_start
        self.metadata: ModelMetadata = metadata

    @classmethod
    def load(cls, path) -> "GgufSource":
        path = os.fspath(path)
        with open(path, "rb") as f:
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        c = _Cursor(mm)
        if c.unpack("<I") != GGUF_MAGIC:
            raise ModelError("gguf: bad magic")
        version = c.unpack("<I")
        if version not in (2, 3):
            raise ModelError(f"gguf: unsupported version {version}")
        n_tensors, n_kv = c.unpack("<Q"), c.unpack("<Q")
        kv = {}
        for _ in range(n_kv):
            key = c.string()
            kv[key] = _read_value(c, c.unpack("<I"))
        tensors = {}
        for _ in range(n_tensors):
            name = c.string()
            nd = c.unpack("<I")
            dims = [c.unpack("<Q") for _ in range(nd)]
            ggml_type, offset = c.unpack("<I"), c.unpack("<Q")
            tensors[name] = TensorInfo(name, dims, ggml_type, offset)
        align = kv.get("general.alignment", 32)
        align = align if isinstance(align, int) and align > 0 else 32
        data_start = -(-c.pos // align) * align
        count = kv.get("split.count")
        if isinstance(count, int) and count > 1:
            no = kv.get("split.no", 0) + 1
            raise ModelError(f"split GGUF: this file is shard {no} of {count}; multi-file GGUF loading "
                             "is not supported")
        md = cls._metadata(kv)
        md.tie_word_embeddings = "output.weight" not in tensors
        return cls(path, mm, kv, tensors, data_start, md)

    @staticmethod
    def _metadata(kv) -> ModelMetadata:
        """build_model_metadata (gguf.rs:331-398), path-relevant fields."""
        arch = kv.get("general.architecture")
        if not isinstance(arch, str):
            raise ModelError("gguf: missing general.architecture")

        def field(name, default=None, required=False):
            v = kv.get(f"{arch}.{name}")
            if isinstance(v, bool) or not isinstance(v, int):
                if required:
                    raise ModelError(f"gguf: missing {name}")
                return default
            return v

        hidden = field("embedding_length", required=True)
        heads = field("attention.head_count", required=True)
        tokens = kv.get("tokenizer.ggml.tokens")
        vocab = field("vocab_size", len(tokens) if isinstance(tokens, list) else 0)
        eos = kv.get("tokenizer.ggml.eos_token_id")
        bos = kv.get("tokenizer.ggml.bos_token_id")
        return ModelMetadata(
            architecture=arch, hidden_size=hidden,
            intermediate_size=field("feed_forward_length", hidden * 4),
            num_hidden_layers=field("block_count", required=True),
            num_attention_heads=heads,
            num_key_value_heads=field("attention.head_count_kv", heads),
            head_dim=field("attention.key_length", hidden // heads),
            max_position_embeddings=field("context_length", 2048),
            vocab_size=vocab,
            eos_token_ids=[eos] if isinstance(eos, int) else [],
            bos_token_id=bos if isinstance(bos, int) else None)

    # -- names -----------------------------------------------------------------
    def tensor_names(self) -> List[str]:
        """HF names of the mapped tensors (plus phi3's fused q/k/v slices)."""
        arch = self.metadata.architecture
        out = [h for h in (map_tensor_name(k, arch) for k in self.tensors) if h]
        if arch == "phi3":
            for k in self.tensors:
                if k.startswith("blk.") and k.endswith(".attn_qkv.weight"):
                    layer = k.split(".")[1]
                    out += [f"model.layers.{layer}.self_attn.{p}_proj.weight" for p in "qkv"]
                    out.append(f"model.layers.{layer}.mlp.gate_proj.weight")
        return sorted(set(out))

    def _fused_slice(self, name: str) -> Optional[Tuple[str, int, int]]:
        """phi3 fused projections (gguf.rs:1034-1059): [q|k|v] rows in
        attn_qkv, [gate|up] rows in ffn_up -> (ggml name, row start, rows)."""
        md = self.metadata
        if md.architecture != "phi3" or not name.startswith("model.layers."):
            return None
        layer, _, rest = name[len("model.layers."):].partition(".")
        q_rows = md.num_attention_heads * md.head_dim
        kv_rows = md.num_key_value_heads * md.head_dim
        ffn = md.intermediate_size
        table = {"self_attn.q_proj.weight": ("attn_qkv.weight", 0, q_rows),
                 "self_attn.k_proj.weight": ("attn_qkv.weight", q_rows, kv_rows),
                 "self_attn.v_proj.weight": ("attn_qkv.weight", q_rows + kv_rows, kv_rows),
                 "mlp.gate_proj.weight": ("ffn_up.weight", 0, ffn),
                 "mlp.up_proj.weight": ("ffn_up.weight", ffn, ffn)}
        if rest not in table:
            return None
        fused, start, rows = table[rest]
        return f"blk.{layer}.{fused}", start, rows

    def _resolve(self, name: str):
        """resolve_tensor (gguf.rs:1061-1078)."""
        fs = self._fused_slice(name)
        if fs is not None and fs[0] in self.tensors:
            return self.tensors[fs[0]], (fs[1], fs[2])
        arch = self.metadata.architecture
        for k, info in self.tensors.items():
            if map_tensor_name(k, arch) == name:
                return info, None
        return None, None

    def _depermute_heads(self, ggml_name: str) -> Optional[int]:
        """Head count to de-permute with (gguf.rs:1080-1094): llama/mistral
        attn_q / attn_k weights and biases."""
        if self.metadata.architecture not in ("llama", "mistral") or not ggml_name.startswith("blk."):
            return None
        rest = ggml_name.split(".", 2)[2] if ggml_name.count(".") >= 2 else ""
        if rest in ("attn_q.weight", "attn_q.bias"):
            return self.metadata.num_attention_heads
        if rest in ("attn_k.weight", "attn_k.bias"):
            return self.metadata.num_key_value_heads
        return None

    # -- the quantized tensor ------------------------------------------------------
    def open_tensor_quant(self, name: str) -> Optional[QuantTensor]:
        """ModelSource::open_tensor_quant (gguf.rs:1233-1289)."""
        info, rows = self._resolve(name)
        if info is None:
            return None
        fmt = _GGML_QUANT.get(info.ggml_type)
        if fmt is None:
            return None
        shape = list(reversed(info.dims))  # HF order: [n_out, k]
        n_elems = int(np.prod(info.dims)) if info.dims else 1
        k_inner = info.dims[0] if info.dims else 1
        size = tensor_byte_size(fmt, n_elems // k_inner, k_inner)
        start = self.data_start + info.offset
        if start + size > len(self._mm):
            raise ModelError(f"gguf tensor {info.name} out of bounds")
        data = memoryview(self._mm)[start:start + size]
        if rows is not None:
            total = max(shape[0], 1)
            if size % total:
                return None
            row_bytes = size // total
            row_start, row_len = rows
            shape[0] = row_len
            data = data[row_start * row_bytes:(row_start + row_len) * row_bytes]
            size = row_len * row_bytes
        n_head = self._depermute_heads(info.name)
        if n_head is not None:
            total = max(shape[0], 1)
            if size % total:
                return None
            row_bytes = size // total
            src = rope_depermute_src_rows(total, n_head)
            packed = np.frombuffer(data, np.uint8).reshape(total, row_bytes)
            data = packed[src].tobytes()
        return QuantTensor(fmt, shape, data)

    def close(self):
        self._mm.close()
