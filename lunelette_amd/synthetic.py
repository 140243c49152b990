"""Host copies of the seeded synthetic model (the bytes the runtime uploads).

Tensor ids follow the reference's weight slots (src/metal_weights.h,
include/model_facts.h): 0 embedding, 1 final norm, then 2 + 9*layer +
{0 input_layernorm, 1 q, 2 k, 3 v, 4 o, 5 post_attention_layernorm, 6 gate,
7 up, 8 down}. Generation runs in the library (lh_synth_*), so these arrays
are bit-identical to what lunelette_metal_create_synthetic uploads.
"""
import ctypes

import numpy as np

from . import HIDDEN, INNER, KV, QUERY, VOCAB, lib

PROJECTIONS = (("q", QUERY, HIDDEN, 1), ("k", KV, HIDDEN, 2), ("v", KV, HIDDEN, 3),
               ("o", HIDDEN, QUERY, 4), ("gate", INNER, HIDDEN, 6), ("up", INNER, HIDDEN, 7),
               ("down", HIDDEN, INNER, 8))


def tensor_id(layer, slot):
    return 2 + 9 * layer + slot


def fp8(seed, tensor, rows, cols, offset=0):
    out = np.empty(rows * cols, dtype=np.uint8)
    lib().lh_synth_fp8(seed, tensor, offset, out.ctypes.data, out.size)
    return out.reshape(rows, cols)


def normal_f32(seed, tensor, n, mean=0.0, std=1.0, offset=0):
    out = np.empty(n, dtype=np.float32)
    lib().lh_synth_normal_f32(seed, tensor, offset, mean, std, out.ctypes.data, n)
    return out


def normal_bf16(seed, tensor, n, mean=0.0, std=1.0, offset=0):
    out = np.empty(n, dtype=np.uint16)
    lib().lh_synth_normal_bf16(seed, tensor, offset, mean, std, out.ctypes.data, n)
    return out


def scale(seed, tensor):
    return float(lib().lh_synth_scale(seed, tensor))


def tokens(seed, stream_id, n):
    out = np.empty(n, dtype=np.int64)
    lib().lh_synth_tokens(seed, stream_id, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), n)
    return out


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def layer(seed, index):
    """Dict of one layer's host tensors: FP8 codes, scales, BF16 norms."""
    out = {"input_norm": normal_bf16(seed, tensor_id(index, 0), HIDDEN, 1.0, 0.02),
           "post_norm": normal_bf16(seed, tensor_id(index, 5), HIDDEN, 1.0, 0.02)}
    for name, rows, cols, slot in PROJECTIONS:
        out[name] = fp8(seed, tensor_id(index, slot), rows, cols)
        out["scale_" + name] = scale(seed, tensor_id(index, slot))
    return out


def embedding(seed):
    return normal_bf16(seed, 0, VOCAB * HIDDEN, 0.0, 0.02).reshape(VOCAB, HIDDEN)


def final_norm(seed):
    return normal_bf16(seed, 1, HIDDEN, 1.0, 0.02)
