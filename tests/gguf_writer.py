"""Minimal GGUF v2/v3 writer for the loader tests (the file layout hearth-gguf
gguf.rs:138-218 reads): magic, version, tensor count, metadata count, typed
key/value pairs, the tensor table, padding to the alignment (v3), tensor data.
"""
import struct

import numpy as np

# GGUF metadata value types (meta.rs MetaValue)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}

# (elements per block, bytes per block) of the ggml types the tests write
BLOCKS = {0: (1, 4), 1: (1, 2), 8: (32, 34), 41: (128, 18), 42: (128, 34), 43: (128, 18), 142: (128, 34),
          143: (128, 28)}


def tensor_nbytes(ggml_type: int, shape) -> int:
    el = int(np.prod(shape, dtype=np.int64))
    be, bb = BLOCKS[ggml_type]
    return (el + be - 1) // be * bb


def _value(vtype, v) -> bytes:
    if vtype == STRING:
        b = v.encode() if isinstance(v, str) else bytes(v)
        return struct.pack("<Q", len(b)) + b
    if vtype == ARRAY:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def write_gguf(path, meta, tensors, version=3, alignment=None, magic=b"GGUF"):
    """meta: [(key, vtype, value)]; tensors: [(name, ggml_type, shape (ne0 first), bytes)].

    With alignment=None the default of 32 applies (no general.alignment key);
    tensor data offsets are multiples of the alignment."""
    align = alignment or 32
    meta = list(meta)
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
    out = bytearray()
    out += magic + struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, vtype, v in meta:
        out += _value(STRING, key) + struct.pack("<I", vtype) + _value(vtype, v)
    offsets, off = [], 0
    for name, t, shape, data in tensors:
        assert len(data) == tensor_nbytes(t, shape), name
        offsets.append(off)
        off += len(data)
        off = (off + align - 1) // align * align
    for (name, t, shape, data), o in zip(tensors, offsets):
        out += _value(STRING, name) + struct.pack("<I", len(shape))
        out += b"".join(struct.pack("<Q", int(d)) for d in shape)
        out += struct.pack("<IQ", t, o)
    if version == 3:
        out += b"\0" * ((align - len(out) % align) % align)
    data_offset = len(out)
    for (name, t, shape, data), o in zip(tensors, offsets):
        out += b"\0" * (data_offset + o - len(out))
        out += data
    with open(path, "wb") as f:
        f.write(out)
    return data_offset, offsets


def model_meta(cfg, arch=None, context_length=None, vocab_as_tokens=False):
    """The metadata a Bonsai-style GGUF carries for a hearth_amd ModelConfig."""
    arch = arch or ("qwen35" if cfg.arch == 1 else "qwen3")
    m = [("general.architecture", STRING, arch),
         (f"{arch}.embedding_length", U32, cfg.d_model),
         (f"{arch}.block_count", U32, cfg.n_layers),
         (f"{arch}.attention.head_count", U32, cfg.n_heads),
         (f"{arch}.attention.head_count_kv", U32, cfg.n_kv_heads),
         (f"{arch}.attention.key_length", U32, cfg.head_dim),
         (f"{arch}.feed_forward_length", U32, cfg.d_ffn),
         (f"{arch}.context_length", U32, context_length or cfg.max_seq),
         (f"{arch}.rope.freq_base", F32, cfg.rope_theta),
         (f"{arch}.rope.dimension_count", U32, cfg.rope_dim or cfg.head_dim),
         (f"{arch}.attention.layer_norm_rms_epsilon", F32, cfg.eps)]
    if vocab_as_tokens:
        m.append(("tokenizer.ggml.tokens", ARRAY, (STRING, [f"t{i}" for i in range(cfg.vocab)])))
    else:
        m.append(("llama.vocab_size", U32, cfg.vocab))
    if cfg.arch == 1:
        m += [(f"{arch}.ssm.state_size", U32, cfg.ssm_head_dim),
              (f"{arch}.ssm.group_count", U32, cfg.ssm_n_k_heads),
              (f"{arch}.ssm.time_step_rank", U32, cfg.ssm_n_v_heads),
              (f"{arch}.ssm.conv_kernel", U32, cfg.ssm_conv_kernel),
              (f"{arch}.ssm.inner_size", U32, cfg.ssm_head_dim * cfg.ssm_n_v_heads),
              (f"{arch}.full_attention_interval", U32, cfg.full_attn_interval)]
    return m


def hadamard_meta(block, signs, version=1, latent=False, tied=False, transform="normalized-sylvester-walsh-hadamard"):
    """prism.hadamard.* keys (qwen35.rs:532-610): signs = {width: +-1 array}."""
    widths = list(signs)
    values = [int(v) for w in widths for v in signs[w]]
    m = [("prism.hadamard.block_size", U32, block), ("prism.hadamard.version", U32, version),
         ("prism.hadamard.transform", STRING, transform),
         ("prism.hadamard.sign_widths", ARRAY, (U32, widths)),
         ("prism.hadamard.sign_values", ARRAY, (I8, values))]
    if latent:
        m.append(("prism.hadamard.inverse_weight_names", ARRAY, (STRING, ["token_embd.weight"])))
    if tied:
        m.append(("prism.hadamard.tied_output", BOOL, 1))
    return m
