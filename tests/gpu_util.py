"""Helpers for GPU tests: device copies of one synthetic layer and of the KV
cache in the device layout [8][capacity][128]."""
import numpy as np

import lunelette_amd as lh
from lunelette_amd import synthetic as syn

import oracle_lib


def decode_table():
    o = oracle_lib.load()
    return np.array([o.orc_fp8_decode(c) for c in range(256)], np.float32)


class DeviceLayer:
    """One layer's weights on device (compact FP8 and resident FP32)."""

    def __init__(self, host, resident=False):
        self.keep = []
        qkv = np.concatenate([host["q"], host["k"], host["v"]], axis=0)
        w = lh.LayerWeights()
        names = ("qkv", "o", "gate", "up", "down")
        mats = {"qkv": qkv, "o": host["o"], "gate": host["gate"], "up": host["up"],
                "down": host["down"]}
        for name in names:
            buf = lh.DeviceBuffer.from_array(mats[name])
            self.keep.append(buf)
            setattr(w, name, buf.ptr)
        if resident:
            # Resident strategy: exact FP32 decode, scale applied per row total.
            dec = decode_table()
            mats32 = {"qkv": dec[qkv]}
            for n in ("o", "gate", "up", "down"):
                mats32[n] = dec[host[n]]
            for name in names:
                buf = lh.DeviceBuffer.from_array(mats32[name].astype(np.float32))
                self.keep.append(buf)
                setattr(w, "f32_" + name, buf.ptr)
        for j, n in enumerate(("q", "k", "v", "o", "gate", "up", "down")):
            w.scale[j] = host["scale_" + n]
        for n in ("input_norm", "post_norm"):
            buf = lh.DeviceBuffer.from_array(syn.bf16_to_f32(host[n]))
            self.keep.append(buf)
            setattr(w, n, buf.ptr)
        self.weights = w


def kv_to_device_layout(kpm, capacity, tail=0.0):
    """[n][1024] position-major -> [8][capacity][128] head-major; rows past n
    hold `tail`."""
    n = kpm.shape[0]
    out = np.full((8, capacity, 128), tail, np.float32)
    out[:, :n] = kpm.reshape(n, 8, 128).transpose(1, 0, 2)
    return out


def kv_from_device_layout(khm, position, count):
    return np.ascontiguousarray(khm[:, position:position + count].transpose(1, 0, 2)).reshape(
        count, 1024)


def k_tiles(khm):
    """[8][capacity][128] head-major K -> the device's tiled K: inside each
    64-position tile, dims 32q + 4i .. +3 of position p at 16-byte word
    ((p // 16) * 8 + i) * 64 + (p % 16) * 4 + q (lh_ktile_word)."""
    h, c, _ = khm.shape
    t = khm.reshape(h, c // 64, 4, 16, 4, 8, 4)        # head, tile, p//16, p%16, q, i, float
    return np.ascontiguousarray(t.transpose(0, 1, 2, 5, 3, 4, 6)).reshape(h, c, 128)


def k_untile(tiled):
    """Inverse of k_tiles."""
    h, c, _ = tiled.shape
    t = tiled.reshape(h, c // 64, 4, 8, 16, 4, 4)      # head, tile, p//16, i, p%16, q, float
    return np.ascontiguousarray(t.transpose(0, 1, 2, 4, 5, 3, 6)).reshape(h, c, 128)


def keys_to_device(kpm, capacity, tail=0.0):
    """Position-major K rows -> the device's K cache layout."""
    return k_tiles(kv_to_device_layout(kpm, capacity, tail))


def attention_on_device(gpu, entry, q, kpm, vpm, length, count, capacity, tail=0.0):
    """Run an attention entry point (lh_attention or lh_attention_mfma) on
    position-major q/K/V (cache rows past them hold `tail`); returns
    [count][4096] and checks the output guard."""
    ws = gpu.lh_workspace_create(capacity, count)
    assert ws, lh.last_error()
    try:
        ids = np.zeros(count, np.int64)
        lh.check(gpu.lh_workspace_set_tokens(ws, ids.ctypes.data_as(lh.c_int64_p), length, count,
                                             None))
        d_q = lh.DeviceBuffer.from_array(q)
        keys = lh.DeviceBuffer.from_array(keys_to_device(kpm, capacity, tail))
        values = lh.DeviceBuffer.from_array(kv_to_device_layout(vpm, capacity, tail))
        out = lh.DeviceBuffer(count * 4096 * 4 + 16)
        lh.check(gpu.lh_memset_device(out.ptr, 0x5a, out.nbytes))
        lh.check(entry(d_q.ptr, keys.ptr, values.ptr, ws, out.ptr, None))
        raw = out.download(np.uint8)
        assert np.all(raw[count * 4096 * 4:] == 0x5a), "wrote past the output"
        return raw[:count * 4096 * 4].view(np.float32)
    finally:
        gpu.lh_workspace_destroy(ws)
