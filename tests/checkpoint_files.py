"""Writers for safetensors test files: small hand-built containers and the
full Ministral-3B-shaped FP8 checkpoint layout (sparse for the CPU contract
tests, or filled with the seeded synthetic model for the GPU load test).
Test infrastructure."""
import json
import os
import struct

import numpy as np

HIDDEN, QUERY, KV, INNER, LAYERS, VOCAB = 3072, 4096, 1024, 9216, 26, 131072

BLOCK = [("input_layernorm.weight", HIDDEN, 0), ("self_attn.q_proj.weight", QUERY, HIDDEN),
         ("self_attn.k_proj.weight", KV, HIDDEN), ("self_attn.v_proj.weight", KV, HIDDEN),
         ("self_attn.o_proj.weight", HIDDEN, QUERY), ("post_attention_layernorm.weight", HIDDEN, 0),
         ("mlp.gate_proj.weight", INNER, HIDDEN), ("mlp.up_proj.weight", INNER, HIDDEN),
         ("mlp.down_proj.weight", HIDDEN, INNER)]
SIZE = {"F8_E4M3": 1, "BF16": 2, "F32": 4, "I64": 8}


def write_container(path, header_text, data=b""):
    """8-byte little-endian header length, the header bytes, the data bytes."""
    raw = header_text.encode("latin-1") if isinstance(header_text, str) else header_text
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(raw)))
        f.write(raw)
        f.write(data)


def slot_tensors():
    """(slot, name, dtype, shape) in the reference slot order."""
    out = [(0, "language_model.model.embed_tokens.weight", "BF16", [VOCAB, HIDDEN]),
           (1, "language_model.model.norm.weight", "BF16", [HIDDEN])]
    for layer in range(LAYERS):
        for i, (suffix, rows, cols) in enumerate(BLOCK):
            name = "language_model.model.layers.%d.%s" % (layer, suffix)
            if cols:
                out.append((2 + 9 * layer + i, name, "F8_E4M3", [rows, cols]))
            else:
                out.append((2 + 9 * layer + i, name, "BF16", [rows]))
    return out


def model_entries(scales):
    """[(name, dtype, shape, payload-or-None)] for the whole checkpoint, data
    order = list order. scales: {slot: (weight_scale_inv bf16 bits,
    activation_scale bf16 bits)} for the FP8 slots."""
    entries = []
    for slot, name, dtype, shape in slot_tensors():
        entries.append([name, dtype, shape, None, slot])
        if dtype == "F8_E4M3":
            prefix = name[:-len("weight")]
            w, a = scales[slot]
            entries.append([prefix + "weight_scale_inv", "BF16", [], struct.pack("<H", w), None])
            entries.append([prefix + "activation_scale", "BF16", [], struct.pack("<H", a), None])
    return entries


def header_for(entries):
    """Header JSON with data_offsets assigned in list order; returns (text, sizes)."""
    header, offset, sizes = {}, 0, []
    for name, dtype, shape, _payload, _slot in entries:
        n = SIZE[dtype]
        for d in shape:
            n *= d
        header[name] = {"dtype": dtype, "shape": shape, "data_offsets": [offset, offset + n]}
        sizes.append(n)
        offset += n
    return json.dumps(header, separators=(",", ":")), sizes


def write_sparse_model(path, entries):
    """Header plus the scalar payloads; every other byte is left as a hole."""
    text, sizes = header_for(entries)
    raw = text.encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(raw)))
        f.write(raw)
        base = 8 + len(raw)
        offset = 0
        for entry, n in zip(entries, sizes):
            if entry[3] is not None:
                f.seek(base + offset)
                f.write(entry[3])
            offset += n
        f.truncate(base + offset)


def bf16_bits(x):
    return int(np.array([x], np.float32).view(np.uint32)[0] >> 16)


def write_synthetic_model(path, lh, seed, chunk=1 << 26):
    """The seeded synthetic model (the bytes lunelette_metal_create_synthetic
    uploads) as a full checkpoint file. Returns the file size."""
    lib = lh.lib()
    scales = {}
    for slot, _name, dtype, _shape in slot_tensors():
        if dtype == "F8_E4M3":
            s = lib.lh_synth_scale(seed, slot)
            scales[slot] = (bf16_bits(s), bf16_bits(1.0))
    entries = model_entries(scales)
    text, sizes = header_for(entries)
    raw = text.encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(raw)))
        f.write(raw)
        for (name, dtype, shape, payload, slot), n in zip(entries, sizes):
            if payload is not None:
                f.write(payload)
                continue
            count = n // SIZE[dtype]
            for begin in range(0, count, chunk):
                m = min(chunk, count - begin)
                if dtype == "F8_E4M3":
                    buf = np.empty(m, np.uint8)
                    lib.lh_synth_fp8(seed, slot, begin, buf.ctypes.data, m)
                else:
                    buf = np.empty(m, np.uint16)
                    mean = 0.0 if slot == 0 else 1.0
                    lib.lh_synth_normal_bf16(seed, slot, begin, mean, 0.02, buf.ctypes.data, m)
                f.write(buf.tobytes())
        return f.tell()
