"""ctypes access to the CPU oracle (oracle/liboracle.so) and, when built, the
reference's own portable C (oracle/_ref/libref.so). Test infrastructure."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle", "liboracle.so")
REFLIB = os.path.join(ROOT, "oracle", "_ref", "libref.so")

REF, MIRROR = 0, 1
W_FP8, W_BF16, W_F32 = 0, 1, 2
LAYERS = 26

c_size = ctypes.c_size_t
c_void = ctypes.c_void_p
c_f = ctypes.c_float


class Layer(ctypes.Structure):
    _fields_ = [("input_norm", c_void), ("post_norm", c_void), ("q", c_void), ("k", c_void),
                ("v", c_void), ("o", c_void), ("gate", c_void), ("up", c_void), ("down", c_void),
                ("scale", c_f * 7)]


class Model(ctypes.Structure):
    _fields_ = [("embedding", c_void), ("final_norm", c_void), ("layers", Layer * LAYERS),
                ("layer_count", c_size), ("capacity", c_size), ("keys", c_void),
                ("values", c_void)]


_lib = None
_ref = None


def _p(lib, name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE):
            raise RuntimeError("oracle/liboracle.so is not built (make -C oracle)")
        _lib = load_path(ORACLE)
    return _lib


def load_path(path):
    """An oracle build at `path` (the shipped one, or a planted-mistake variant
    a test compiled) with its prototypes declared."""
    l = ctypes.CDLL(path)
    i = ctypes.c_int
    fp = ctypes.POINTER(c_f)
    _p(l, "orc_fp8_decode", c_f, ctypes.c_uint8)
    _p(l, "orc_bf16_widen", c_f, ctypes.c_uint16)
    _p(l, "orc_bf16_round", ctypes.c_uint16, c_f)
    _p(l, "orc_yarn", i, ctypes.c_uint32, fp, fp)
    _p(l, "orc_query_factor", c_f, ctypes.c_uint32)
    _p(l, "orc_select_greedy", i, c_void, c_size, ctypes.POINTER(ctypes.c_int64))
    _p(l, "orc_expf", c_f, c_f)
    _p(l, "orc_silu_ref", c_f, c_f)
    _p(l, "orc_silu_mirror", c_f, c_f)
    _p(l, "orc_matvec", None, i, i, c_void, c_f, c_void, c_void, c_size, c_size, c_size)
    _p(l, "orc_rmsnorm", None, i, c_void, c_void, c_void, c_size, c_size)
    _p(l, "orc_rope", None, c_void, c_void, c_void, c_void, c_void, c_size, c_size)
    _p(l, "orc_silu_mul", None, i, c_void, c_void, c_void, c_size)
    _p(l, "orc_attention", None, i, c_void, c_void, c_void, c_size, c_size, c_size, c_size,
       c_void)
    _p(l, "orc_layer_forward", None, i, ctypes.POINTER(Model), c_size, c_void, c_size, c_size)
    _p(l, "orc_model_forward", i, i, ctypes.POINTER(Model), c_void, c_size, c_size, c_void)
    _p(l, "orc_set_threads", None, i)
    _p(l, "orc_get_threads", i)
    return l


PLANTS = {1: "attention residual skipped", 2: "post-norm fed x instead of x+o",
          3: "query factor on K instead of Q", 4: "V rotated before caching",
          5: "head on row 0", 6: "K cached unrotated", 7: "MLP residual on the layer input",
          8: "query factor dropped"}


def build_planted(plants, directory):
    """Oracle builds with one planted composition mistake each (orc_model.c
    compiled with -DORC_PLANT=n), compiled in parallel into `directory`;
    returns {n: library}."""
    import subprocess
    src = os.path.join(ROOT, "oracle")
    procs = {}
    for n in plants:
        lib = os.path.join(str(directory), "liboracle_plant%d.so" % n)
        cmd = ["gcc", "-std=c11", "-O3", "-march=x86-64-v3", "-ffp-contract=off",
               "-fno-math-errno", "-fopenmp", "-fPIC", "-shared", "-DORC_PLANT=%d" % n,
               os.path.join(src, "orc_basic.c"), os.path.join(src, "orc_kernels.c"),
               os.path.join(src, "orc_model.c"), "-o", lib, "-lm"]
        procs[n] = (subprocess.Popen(cmd, stderr=subprocess.PIPE), lib)
    libs = {}
    for n, (proc, lib) in procs.items():
        _, err = proc.communicate()
        if proc.returncode != 0:
            raise RuntimeError(err.decode())
        libs[n] = load_path(lib)
    return libs


def load_ref():
    """The reference's own C (safetensors container, checkpoint contract, FP8/BF16
    decode, YaRN, greedy), or None."""
    global _ref
    if _ref is None and os.path.exists(REFLIB):
        l = ctypes.CDLL(REFLIB)
        fp = ctypes.POINTER(c_f)
        _p(l, "st_f8_e4m3_to_f32", c_f, ctypes.c_ubyte)
        _p(l, "st_bf16_to_f32", c_f, ctypes.c_uint16)
        _p(l, "lunelette_metal_yarn", ctypes.c_int, ctypes.c_uint32, fp, fp)
        _p(l, "lunelette_select_greedy", ctypes.c_int, c_void, ctypes.POINTER(ctypes.c_int64),
           ctypes.c_char_p, c_size)
        _ref = l
    return _ref


def ptr(a):
    return a.ctypes.data


def matvec(schedule, kind, w, scale, x, rows, cols, tokens=1):
    y = np.empty(tokens * rows, dtype=np.float32)
    load().orc_matvec(schedule, kind, ptr(w), scale, ptr(np.ascontiguousarray(x, np.float32)),
                      ptr(y), rows, cols, tokens)
    return y


def rmsnorm(schedule, gamma, x, width, tokens=1):
    out = np.empty(width * tokens, dtype=np.float32)
    load().orc_rmsnorm(schedule, ptr(gamma), ptr(x), ptr(out), width, tokens)
    return out


def attention(schedule, q, keys, values, head_stride, pos_stride, prefix, count):
    out = np.empty(count * 4096, dtype=np.float32)
    load().orc_attention(schedule, ptr(q), ptr(keys), ptr(values), head_stride, pos_stride,
                         prefix, count, ptr(out))
    return out


def yarn(position):
    c = np.empty(128, dtype=np.float32)
    s = np.empty(128, dtype=np.float32)
    fp = ctypes.POINTER(c_f)
    rc = load().orc_yarn(position, c.ctypes.data_as(fp), s.ctypes.data_as(fp))
    return rc, c, s


class HostModel:
    """Oracle model over host arrays (keeps the arrays alive)."""

    def __init__(self, embedding, final_norm, layers, capacity, lib=None):
        self.lib = lib
        self.keep = [embedding, final_norm]
        self.keys = np.zeros(len(layers) * 8 * capacity * 128, dtype=np.float32)
        self.values = np.zeros_like(self.keys)
        m = Model()
        m.embedding = ptr(embedding)
        m.final_norm = ptr(final_norm)
        for i, layer in enumerate(layers):
            L = m.layers[i]
            for name in ("input_norm", "post_norm", "q", "k", "v", "o", "gate", "up", "down"):
                setattr(L, name, ptr(layer[name]))
                self.keep.append(layer[name])
            for j, name in enumerate(("q", "k", "v", "o", "gate", "up", "down")):
                L.scale[j] = layer["scale_" + name]
        m.layer_count = len(layers)
        m.capacity = capacity
        m.keys = ptr(self.keys)
        m.values = ptr(self.values)
        self.model = m
        self.capacity = capacity

    def forward(self, schedule, ids, length):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        logits = np.empty(131072, dtype=np.float32)
        rc = (self.lib or load()).orc_model_forward(schedule, ctypes.byref(self.model), ptr(ids), length,
                                      len(ids), ptr(logits))
        if rc:
            raise RuntimeError("oracle forward rejected")
        return logits

    def layer_forward(self, schedule, layer, x, length, count):
        (self.lib or load()).orc_layer_forward(schedule, ctypes.byref(self.model), layer, ptr(x), length, count)

    def kv(self, layer, kind, position, count):
        """[count][1024] rows in the reference's position-major layout."""
        cache = self.values if kind else self.keys
        C = self.capacity
        base = cache[layer * 8 * C * 128:(layer + 1) * 8 * C * 128].reshape(8, C, 128)
        return np.ascontiguousarray(base[:, position:position + count, :].transpose(1, 0, 2)
                                    ).reshape(count, 1024)
