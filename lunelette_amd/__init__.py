"""Python bindings (ctypes) for the gfx950 Lunelette forward path.

The product is the C-ABI shared library lunelette_amd/liblunelette_hip.so
(include/lunelette_runtime.h, include/lunelette_kernels.h,
include/lunelette_generation.h, include/lunelette_session.h,
include/lunelette_artifacts.h, include/lunelette_tokenizer.h,
include/lunelette_chat.h). This module only loads it and declares
prototypes; it never substitutes another implementation. If the library has
not been built, `lib()` raises.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(_HERE, "liblunelette_hip.so")
# The same objects plus the host-forced failure seams (csrc/lh_test_seams.h),
# for the runtime's state-machine tests only.
TEST_LIBRARY = os.path.join(_HERE, "liblunelette_hip_test.so")

VOCAB = 131072
HIDDEN = 3072
QUERY = 4096
KV = 1024
INNER = 9216
LAYERS = 26
QKV_ROWS = QUERY + 2 * KV

PREFILL_MPS = 0
PREFILL_CUSTOM = 1
RESIDENT_FP32 = 0
COMPACT_FP8_ARITHMETIC = 1
COMPACT_FP8_LOOKUP = 2

PATH_FUSED, PATH_LOOKUP, PATH_UNFUSED, PATH_RESIDENT, PATH_MFMA = range(5)
OP_QKV_ROPE, OP_ATTENTION, OP_O_RESIDUAL, OP_GATEUP_SILU, OP_DOWN_RESIDUAL = range(5)

_lib = None
_test_lib = None

c_size = ctypes.c_size_t
c_void = ctypes.c_void_p
c_float_p = ctypes.POINTER(ctypes.c_float)
c_int64_p = ctypes.POINTER(ctypes.c_int64)


class Options(ctypes.Structure):
    _fields_ = [("prefill", ctypes.c_int), ("strategy", ctypes.c_int)]


class Limits(ctypes.Structure):
    _fields_ = [("context", c_size), ("block", c_size)]


class Memory(ctypes.Structure):
    _fields_ = [("strategy", ctypes.c_int), ("weight_bytes", ctypes.c_uint64),
                ("conversion_stage_bytes", ctypes.c_uint64), ("scratch_bytes", ctypes.c_uint64),
                ("kv_bytes", ctypes.c_uint64), ("total_bytes", ctypes.c_uint64)]


class SyntheticConfig(ctypes.Structure):
    _fields_ = [("seed", ctypes.c_uint64), ("layers", ctypes.c_uint32)]


class LayerWeights(ctypes.Structure):
    _fields_ = [("qkv", c_void), ("o", c_void), ("gate", c_void), ("up", c_void), ("down", c_void),
                ("f32_qkv", c_void), ("f32_o", c_void), ("f32_gate", c_void), ("f32_up", c_void),
                ("f32_down", c_void), ("scale", ctypes.c_float * 7),
                ("input_norm", c_void), ("post_norm", c_void)]


class GenerationConfig(ctypes.Structure):
    _fields_ = [("max_new_tokens", c_size), ("eos_token", ctypes.c_int64)]


class GenerationResult(ctypes.Structure):
    _fields_ = [("tokens", ctypes.c_int64 * 256), ("count", c_size), ("stop", ctypes.c_int)]


LOGITS_FN = ctypes.CFUNCTYPE(ctypes.c_int, c_void, c_int64_p, c_size, c_float_p,
                             ctypes.c_char_p, c_size)


def _proto(lib, name, restype, *argtypes):
    fn = getattr(lib, name)
    fn.restype = restype
    fn.argtypes = list(argtypes)


def lib():
    """Load the built library (raises if it is missing)."""
    global _lib
    if _lib is None:
        _lib = _load(LIBRARY)
    return _lib


def test_lib():
    """Load the test build (the shipped library's objects plus the failure
    seams of csrc/lh_test_seams.h); raises if it is missing."""
    global _test_lib
    if _test_lib is None:
        l = _load(TEST_LIBRARY)
        i, f = ctypes.c_int, ctypes.c_float
        _proto(l, "lunelette_metal_test_inject", i, c_void, i)
        _proto(l, "lunelette_metal_test_fail_after_layer", i, c_void, ctypes.c_uint32)
        _proto(l, "lunelette_metal_test_set_epoch", i, c_void, ctypes.c_uint64)
        _proto(l, "lunelette_metal_test_set_logit", i, c_void, c_size, f)
        _proto(l, "lunelette_metal_test_chained", i, ctypes.c_uint32)
        _proto(l, "lunelette_metal_test_fail_allocation", None, ctypes.c_uint)
        _proto(l, "lunelette_metal_test_allocations", ctypes.c_uint)
        _proto(l, "lunelette_metal_test_live_allocations", ctypes.c_long)
        _proto(l, "lunelette_metal_test_fail_host_allocation", None, ctypes.c_uint)
        _proto(l, "lunelette_metal_test_host_allocations", ctypes.c_uint)
        _proto(l, "lunelette_metal_test_live_host_allocations", ctypes.c_long)
        _test_lib = l
    return _test_lib


def _load(path):
    if not os.path.exists(path):
        raise RuntimeError("%s is not built; run __graft_entry__.build()" %
                           os.path.basename(path))
    l = ctypes.CDLL(path)
    i, v, f = ctypes.c_int, None, ctypes.c_float
    _proto(l, "lh_last_error", ctypes.c_char_p)
    _proto(l, "lh_device_count", i)
    _proto(l, "lh_device_alloc", c_void, c_size)
    _proto(l, "lh_device_free", v, c_void)
    _proto(l, "lh_host_alloc_pinned", c_void, c_size)
    _proto(l, "lh_host_free_pinned", v, c_void)
    _proto(l, "lh_memcpy_htod", i, c_void, c_void, c_size)
    _proto(l, "lh_memcpy_dtoh", i, c_void, c_void, c_size)
    _proto(l, "lh_memcpy_dtod", i, c_void, c_void, c_size)
    _proto(l, "lh_memset_device", i, c_void, i, c_size)
    _proto(l, "lh_device_synchronize", i)
    _proto(l, "lh_stream_create", c_void)
    _proto(l, "lh_stream_synchronize", i, c_void)
    _proto(l, "lh_stream_destroy", v, c_void)
    _proto(l, "lh_event_create", c_void)
    _proto(l, "lh_event_record", i, c_void, c_void)
    _proto(l, "lh_event_elapsed_ms", i, c_void, c_void, c_float_p)
    _proto(l, "lh_event_destroy", v, c_void)
    _proto(l, "lh_fp8_matvec", i, c_void, f, c_void, c_void, c_size, c_size, c_size, i, c_void)
    _proto(l, "lh_f32_matvec", i, c_void, c_void, c_void, c_size, c_size, c_size, c_void)
    _proto(l, "lh_bf16_matvec", i, c_void, c_void, c_void, c_size, c_size, c_size, c_void)
    _proto(l, "lh_rmsnorm", i, c_void, c_void, c_void, c_size, c_size, c_void)
    _proto(l, "lh_element", i, i, c_void, c_void, c_void, c_size, c_void)
    _proto(l, "lh_read_floor", i, c_void, c_size, ctypes.c_uint, ctypes.c_uint, c_void, c_void)
    _proto(l, "lh_rope", i, c_void, c_void, c_void, c_void, c_void, c_size, c_size, c_void)
    _proto(l, "lh_fp8_decode", i, c_void, c_void, c_size, c_void)
    _proto(l, "lh_expf", i, c_void, c_void, c_size, c_void)
    _proto(l, "lh_workspace_create", c_void, c_size, c_size)
    _proto(l, "lh_workspace_destroy", v, c_void)
    _proto(l, "lh_workspace_set_tokens", i, c_void, c_int64_p, c_size, c_size, c_void)
    _proto(l, "lh_layer_forward", i, ctypes.POINTER(LayerWeights), c_void, c_void, c_void,
           c_void, i, c_void)
    _proto(l, "lh_head_forward", i, c_void, c_void, c_void, c_void, c_void)
    _proto(l, "lh_head_forward_checked", i, c_void, c_void, c_void, c_void, c_void, c_void)
    _proto(l, "lh_fp8_gemm", i, c_void, c_void, f, c_void, c_void, c_size, c_size, c_size, c_void)
    _proto(l, "lh_layer_operator", i, i, ctypes.POINTER(LayerWeights), c_void, c_void, c_void,
           c_void, c_void)
    _proto(l, "lh_attention", i, c_void, c_void, c_void, c_void, c_void, c_void)
    _proto(l, "lh_attention_mfma", i, c_void, c_void, c_void, c_void, c_void, c_void)
    _proto(l, "lh_attention_noalloc", i, c_void, c_void, c_void, c_size, c_size, c_size, c_void,
           c_void)
    _proto(l, "lh_embed_forward", i, c_void, c_void, c_void, c_void)
    _proto(l, "lh_yarn", i, ctypes.c_uint32, c_float_p, c_float_p)
    _proto(l, "lh_query_factor", f, ctypes.c_uint32)
    _proto(l, "lh_synth_fp8", v, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64, c_void, c_size)
    _proto(l, "lh_synth_normal_f32", v, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64, f, f,
           c_void, c_size)
    _proto(l, "lh_synth_normal_bf16", v, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64, f, f,
           c_void, c_size)
    _proto(l, "lh_synth_scale", f, ctypes.c_uint64, ctypes.c_uint32)
    _proto(l, "lh_synth_tokens", v, ctypes.c_uint64, ctypes.c_uint32, c_int64_p, c_size)
    _proto(l, "lh_st_inspect", i, ctypes.c_char_p, ctypes.c_char_p, c_size, ctypes.c_char_p,
           c_size)
    _proto(l, "lh_st_read_tensor", i, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_uint64,
           c_void, c_size, ctypes.c_char_p, c_size)
    _proto(l, "lh_checkpoint_check", i, ctypes.c_char_p, c_float_p, ctypes.c_char_p, c_size)
    _proto(l, "lh_fp8_admit", i, c_void, c_size, f, i, ctypes.c_char_p, c_size)
    err = ctypes.c_char_p
    _proto(l, "lunelette_metal_create", c_void, ctypes.c_char_p, err, c_size)
    _proto(l, "lunelette_metal_create_with_options", c_void, ctypes.c_char_p,
           ctypes.POINTER(Options), err, c_size)
    _proto(l, "lunelette_metal_create_configured", c_void, ctypes.c_char_p,
           ctypes.POINTER(Options), ctypes.POINTER(Limits), err, c_size)
    _proto(l, "lunelette_metal_create_synthetic", c_void, ctypes.POINTER(SyntheticConfig),
           ctypes.POINTER(Options), ctypes.POINTER(Limits), err, c_size)
    _proto(l, "lunelette_metal_get_limits", i, c_void, ctypes.POINTER(Limits))
    _proto(l, "lunelette_metal_get_memory", i, c_void, ctypes.POINTER(Memory))
    _proto(l, "lunelette_metal_destroy", v, c_void)
    _proto(l, "lunelette_metal_reset", i, c_void, err, c_size)
    logits_out = ctypes.POINTER(c_float_p)
    _proto(l, "lunelette_metal_prefill", i, c_void, c_int64_p, c_size, logits_out, err, c_size)
    _proto(l, "lunelette_metal_decode", i, c_void, ctypes.c_int64, logits_out, err, c_size)
    _proto(l, "lunelette_metal_append", i, c_void, c_int64_p, c_size, logits_out, err, c_size)
    _proto(l, "lunelette_metal_checkpoint_create", i, c_void, ctypes.POINTER(c_void), err, c_size)
    _proto(l, "lunelette_metal_checkpoint_restore", i, c_void, c_void, logits_out, err, c_size)
    _proto(l, "lunelette_metal_checkpoint_destroy", v, c_void)
    _proto(l, "lunelette_metal_last_device_ms", i, c_void, c_float_p)
    _proto(l, "lunelette_metal_read_kv", i, c_void, c_size, i, c_size, c_size, c_float_p)
    _proto(l, "lunelette_select_greedy", i, c_float_p, c_int64_p, err, c_size)
    _proto(l, "lunelette_generate_with_logits", i, LOGITS_FN, c_void, c_int64_p, c_size,
           ctypes.POINTER(GenerationConfig), ctypes.POINTER(GenerationResult), err, c_size)
    _proto(l, "lunelette_generate_with_logits_capacity", i, LOGITS_FN, c_void, c_int64_p, c_size,
           c_size, ctypes.POINTER(GenerationConfig), ctypes.POINTER(GenerationResult), err,
           c_size)
    declare_session(l)
    declare_artifacts(l)
    declare_tokenizer(l)
    return l


class SessionWork(ctypes.Structure):
    """lunelette_session_work: the receipt of the last materialize/restore."""
    _fields_ = [(name, ctypes.c_uint) for name in (
        "reused", "full_attempted", "full_committed", "suffix_attempted", "suffix_committed",
        "pending_attempted", "pending_committed", "prefill_calls", "append_calls",
        "decode_calls", "decode_attempted", "decode_committed", "logit_restores",
        "recompute_attempted", "recompute_committed")]


class SessionOptions(ctypes.Structure):
    _fields_ = [("context", c_size), ("block", c_size), ("prefix_reuse", ctypes.c_int),
                ("replay_path", ctypes.c_char_p)]


def declare_session(l):
    """Prototypes of include/lunelette_session.h on a loaded library (the
    product, or a test library that links the adapter with another runtime)."""
    i, u, v = ctypes.c_int, ctypes.c_uint, None
    err = ctypes.c_char_p
    u_p = ctypes.POINTER(ctypes.c_uint)
    _proto(l, "lunelette_session_open", c_void, ctypes.c_char_p, ctypes.POINTER(Options),
           ctypes.POINTER(SessionOptions), err, c_size)
    _proto(l, "lunelette_session_adopt", c_void, c_void, ctypes.POINTER(Options),
           ctypes.POINTER(SessionOptions), err, c_size)
    _proto(l, "lunelette_session_destroy", v, c_void)
    _proto(l, "lunelette_session_materialize", i, c_void, u_p, u)
    _proto(l, "lunelette_session_materialize_step", i, c_void, u_p, u, u_p)
    _proto(l, "lunelette_session_next", i, c_void)
    _proto(l, "lunelette_session_replay_next", i, c_void, u)
    _proto(l, "lunelette_session_save", i, c_void)
    _proto(l, "lunelette_session_restore", i, c_void)
    _proto(l, "lunelette_session_begin", v, c_void)
    _proto(l, "lunelette_session_take_work", v, c_void, ctypes.POINTER(SessionWork))
    _proto(l, "lunelette_session_invalidate", v, c_void)
    _proto(l, "lunelette_session_reset", v, c_void)
    _proto(l, "lunelette_session_length", u, c_void)
    _proto(l, "lunelette_session_context_capacity", u, c_void)
    _proto(l, "lunelette_session_block_capacity", u, c_void)
    _proto(l, "lunelette_session_prefix_reuse", u, c_void)
    _proto(l, "lunelette_session_error", ctypes.c_char_p, c_void)
    _proto(l, "lunelette_session_logits", c_float_p, c_void)
    _proto(l, "lunelette_session_info", ctypes.c_char_p, c_void)


def last_error():
    return lib().lh_last_error().decode()


def require_gpu():
    """Raise unless a HIP device is visible (the product has no CPU path)."""
    if lib().lh_device_count() < 1:
        raise RuntimeError("no HIP device visible: the gfx950 library needs an MI355X")


class DeviceBuffer:
    """Owned device allocation with numpy upload/download."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = lib().lh_device_alloc(self.nbytes)
        if not self.ptr:
            raise MemoryError(last_error())

    @classmethod
    def from_array(cls, array):
        array = np.ascontiguousarray(array)
        buf = cls(array.nbytes)
        buf.upload(array)
        return buf

    def upload(self, array):
        array = np.ascontiguousarray(array)
        assert array.nbytes <= self.nbytes
        if lib().lh_memcpy_htod(self.ptr, array.ctypes.data, array.nbytes):
            raise RuntimeError(last_error())

    def download(self, dtype, count=None):
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        if lib().lh_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes):
            raise RuntimeError(last_error())
        return out

    def free(self):
        if self.ptr:
            lib().lh_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def check(status, what="call"):
    if status != 0:
        raise RuntimeError("%s failed: %s" % (what, last_error()))


class LogitMetrics(ctypes.Structure):
    """lunelette_logit_metrics."""
    _fields_ = [("finite_a", c_size), ("finite_b", c_size), ("exact", ctypes.c_int),
                ("top1_a", c_size), ("top1_b", c_size), ("top5", c_size), ("top20", c_size),
                ("top64", c_size), ("max_abs", ctypes.c_double), ("rms", ctypes.c_double),
                ("cosine", ctypes.c_double)]


class NativeTrajectory(ctypes.Structure):
    """lunelette_native_trajectory."""
    _fields_ = [("magic", ctypes.c_uint32), ("strategy", ctypes.c_int), ("mode", ctypes.c_uint32),
                ("count", c_size), ("ids", ctypes.c_int64 * 248), ("forced", ctypes.c_int64 * 8)]


def declare_artifacts(l):
    """Prototypes of include/lunelette_artifacts.h on a loaded library."""
    i, err = ctypes.c_int, ctypes.c_char_p
    traj = ctypes.POINTER(NativeTrajectory)
    metrics = ctypes.POINTER(LogitMetrics)
    _proto(l, "lunelette_logits_top64", None, c_float_p, c_size, ctypes.POINTER(c_size))
    _proto(l, "lunelette_logits_compare", i, c_float_p, c_float_p, c_size, metrics)
    _proto(l, "lunelette_native_write", i, ctypes.c_char_p, traj, c_float_p, err, c_size)
    _proto(l, "lunelette_native_read", i, ctypes.c_char_p, traj, c_float_p, err, c_size)
    _proto(l, "lunelette_native_compare_files", i, ctypes.c_char_p, ctypes.c_char_p,
           ctypes.c_uint32, c_size, ctypes.c_int, metrics, err, c_size)
    _proto(l, "lunelette_native_run", i, c_void, ctypes.c_char_p, traj, i, metrics, err, c_size)


def declare_tokenizer(l):
    """Prototypes of include/lunelette_tokenizer.h and include/lunelette_chat.h
    (the product, or the reference's tokenizer built from source)."""
    i, err = ctypes.c_int, ctypes.c_char_p
    u32_pp = ctypes.POINTER(ctypes.POINTER(ctypes.c_uint32))
    u8_pp = ctypes.POINTER(ctypes.POINTER(ctypes.c_ubyte))
    size_p = ctypes.POINTER(c_size)
    _proto(l, "lunelette_tokenizer_open", i, ctypes.c_char_p, ctypes.POINTER(c_void), err, c_size)
    _proto(l, "lunelette_tokenizer_close", None, c_void)
    _proto(l, "lunelette_tokenizer_encode", i, c_void, ctypes.c_char_p, c_size, u32_pp, size_p,
           err, c_size)
    _proto(l, "lunelette_tokenizer_encode_with_limit", i, c_void, ctypes.c_char_p, c_size, c_size,
           u32_pp, size_p, err, c_size)
    _proto(l, "lunelette_tokenizer_decode", i, c_void, ctypes.POINTER(ctypes.c_uint32), c_size,
           u8_pp, size_p, err, c_size)
    _proto(l, "lunelette_chat_prompt", i, c_void, ctypes.c_char_p, ctypes.c_char_p, i,
           c_int64_p, size_p, err, c_size)
    if hasattr(l, "lunelette_tokenizer_split"):
        _proto(l, "lunelette_tokenizer_split", ctypes.c_long, ctypes.c_char_p, c_size, size_p,
               c_size)
