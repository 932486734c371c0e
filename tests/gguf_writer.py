"""A GGUF v2/v3 writer for the tests (little-endian, the llama.cpp file layout): header, metadata
key/values, tensor directory, data section aligned to general.alignment. Writes the synthetic model
files the reader and kcModelLoadGguf tests load (no model file ships with the reference)."""
import struct

import numpy as np

# GGUF metadata value types
U8, I8, U16, I16, U32, I32, F32V, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32V: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}
# ggml tensor types
GGML_F32, GGML_F16, GGML_Q4_K, GGML_Q6_K = 0, 1, 12, 14
_BLOCK = {GGML_F32: (4, 1), GGML_F16: (2, 1), GGML_Q4_K: (144, 256), GGML_Q6_K: (210, 256), 8: (34, 32)}


def _s(b):
    b = b.encode() if isinstance(b, str) else b
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _s(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(_FMT[t], v)


def tensor_bytes(ggml_type, ne):
    bb, bv = _BLOCK[ggml_type]
    n = int(np.prod(ne))
    return n // bv * bb


def write_gguf(path, kv, tensors, alignment=32, version=3):
    """kv: [(key, type, value)] (arrays: value = (elem_type, [items])); tensors: [(name, ggml_type,
    ne, bytes-like)] with ne[0] the values per row. Writes general.alignment when it is not 32."""
    kv = list(kv)
    if alignment != 32:
        kv.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, t, v in kv:
        head += _s(key) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for name, gt, ne, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        off += len(bytes(data))
    for (name, gt, ne, data), o in zip(tensors, offs):
        head += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", gt, o)
    pad = (-len(head)) % alignment
    blob = bytearray(head + b"\0" * pad)
    start = len(blob)
    for (name, gt, ne, data), o in zip(tensors, offs):
        d = bytes(data)
        blob += b"\0" * (start + o - len(blob))
        blob += d
    with open(path, "wb") as f:
        f.write(bytes(blob))


# model tensor ids (include/kernelcore/model.h) -> GGUF tensor names
NAMES = {0: "token_embd", 1: "output_norm", 2: "output", 3: "attn_norm", 4: "attn_q", 5: "attn_k", 6: "attn_v",
         7: "attn_output", 8: "ffn_norm", 9: "ffn_gate", 10: "ffn_up", 11: "ffn_down", 12: "attn_q_norm",
         13: "attn_k_norm", 14: "rope_freqs"}


def model_gguf(path, arch, cfg, weights, types, tied=False, extra_kv=()):
    """A model file: weights[(id, layer)] as for kcModelSetTensor (layer -1 for global tensors),
    types[(id, layer)] the ggml type of every matrix. tied: no output.weight."""
    kv = [("general.architecture", STR, arch), ("general.name", STR, "synthetic " + arch),
          (f"{arch}.block_count", U32, cfg["n_layer"]), (f"{arch}.embedding_length", U32, cfg["n_embd"]),
          (f"{arch}.feed_forward_length", U32, cfg["n_ff"]), (f"{arch}.attention.head_count", U32, cfg["n_head"]),
          (f"{arch}.attention.head_count_kv", U32, cfg["n_head_kv"]),
          (f"{arch}.attention.key_length", U32, cfg["head_dim"]),
          (f"{arch}.attention.layer_norm_rms_epsilon", F32V, cfg["norm_eps"]),
          (f"{arch}.rope.freq_base", F32V, cfg["rope_theta"]),
          ("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(16)]))] + list(extra_kv)
    E, Q, KV, F, V = (cfg["n_embd"], cfg["n_head"] * cfg["head_dim"], cfg["n_head_kv"] * cfg["head_dim"],
                      cfg["n_ff"], cfg["n_vocab"])
    shape = {0: (E, V), 1: (E,), 2: (E, V), 3: (E,), 4: (E, Q), 5: (E, KV), 6: (E, KV), 7: (Q, E), 8: (E,),
             9: (E, F), 10: (E, F), 11: (F, E), 12: (cfg["head_dim"],), 13: (cfg["head_dim"],),
             14: (cfg["head_dim"] // 2,)}
    tensors = []
    for (tid, layer), data in sorted(weights.items(), key=lambda kv: (kv[0][1], kv[0][0])):
        if tied and tid == 2:
            continue
        name = NAMES[tid] + ".weight" if layer < 0 else f"blk.{layer}.{NAMES[tid]}.weight"
        gt = types.get((tid, layer), GGML_F32)
        tensors.append((name, gt, shape[tid], np.ascontiguousarray(data).tobytes()))
    write_gguf(path, kv, tensors)
