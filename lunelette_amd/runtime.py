"""Python view of the runtime C-ABI (include/lunelette_runtime.h).

Thin: every call goes to liblunelette_hip.so; errors raise RuntimeError with
the library's diagnostic. Logits are returned as numpy copies of the borrowed
host buffer.
"""
import ctypes

import numpy as np

from . import (COMPACT_FP8_ARITHMETIC, Limits, Memory, Options, PREFILL_MPS, SyntheticConfig,
               VOCAB, c_float_p, c_int64_p, lib, test_lib)


class RuntimeError_(RuntimeError):
    pass


class Runtime:
    """A runtime context over the seeded synthetic model, or over the FP8
    safetensors checkpoint at `path` (lunelette_metal_create_configured; all
    26 layers). seams=True creates it in the test build of the library, whose
    host-forced failure seams the inject/fail_* methods drive."""

    def __init__(self, seed=1, layers=26, context=4352, block=256, prefill=PREFILL_MPS,
                 strategy=COMPACT_FP8_ARITHMETIC, path=None, seams=False):
        self._lib = test_lib() if seams else lib()
        self._err = ctypes.create_string_buffer(512)
        opts = Options(prefill, strategy)
        lim = Limits(context, block)
        if path is None:
            cfg = SyntheticConfig(seed, layers)
            self.handle = self._lib.lunelette_metal_create_synthetic(
                ctypes.byref(cfg), ctypes.byref(opts), ctypes.byref(lim), self._err, 512)
        else:
            layers = 26
            self.handle = self._lib.lunelette_metal_create_configured(
                str(path).encode(), ctypes.byref(opts), ctypes.byref(lim), self._err, 512)
        if not self.handle:
            raise RuntimeError_("create failed: " + self._err.value.decode())
        self.layers, self.context, self.block = layers, context, block
        self.prefill_mode, self.strategy = prefill, strategy
        self._logits = c_float_p()

    def close(self):
        if self.handle:
            self._lib.lunelette_metal_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _result(self, rc, copy):
        if rc != 0:
            raise RuntimeError_(self._err.value.decode())
        if not copy:
            return None
        return np.ctypeslib.as_array(self._logits, shape=(VOCAB,)).copy()

    def prefill(self, ids, copy=True):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        rc = self._lib.lunelette_metal_prefill(self.handle, ids.ctypes.data_as(c_int64_p),
                                               ids.size, ctypes.byref(self._logits), self._err,
                                               512)
        return self._result(rc, copy)

    def append(self, ids, copy=True):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        rc = self._lib.lunelette_metal_append(self.handle, ids.ctypes.data_as(c_int64_p),
                                              ids.size, ctypes.byref(self._logits), self._err,
                                              512)
        return self._result(rc, copy)

    def decode(self, token, copy=True):
        rc = self._lib.lunelette_metal_decode(self.handle, int(token), ctypes.byref(self._logits),
                                              self._err, 512)
        return self._result(rc, copy)

    def greedy(self):
        """Greedy token of the currently borrowed logits (lunelette_select_greedy)."""
        token = ctypes.c_int64(-1)
        if self._lib.lunelette_select_greedy(self._logits, ctypes.byref(token), self._err, 512):
            raise RuntimeError_(self._err.value.decode())
        return token.value

    def reset(self):
        if self._lib.lunelette_metal_reset(self.handle, self._err, 512):
            raise RuntimeError_(self._err.value.decode())

    def checkpoint(self):
        handle = ctypes.c_void_p()
        if self._lib.lunelette_metal_checkpoint_create(self.handle, ctypes.byref(handle),
                                                       self._err, 512):
            raise RuntimeError_(self._err.value.decode())
        return handle.value

    def restore(self, checkpoint, copy=True):
        rc = self._lib.lunelette_metal_checkpoint_restore(self.handle, checkpoint,
                                                          ctypes.byref(self._logits), self._err,
                                                          512)
        return self._result(rc, copy)

    def destroy_checkpoint(self, checkpoint):
        self._lib.lunelette_metal_checkpoint_destroy(checkpoint)

    def memory(self):
        m = Memory()
        if self._lib.lunelette_metal_get_memory(self.handle, ctypes.byref(m)):
            raise RuntimeError_("get_memory failed")
        return {k: getattr(m, k) for k, _ in Memory._fields_}

    def limits(self):
        lim = Limits()
        if self._lib.lunelette_metal_get_limits(self.handle, ctypes.byref(lim)):
            raise RuntimeError_("get_limits failed")
        return lim.context, lim.block

    def last_device_ms(self):
        ms = ctypes.c_float()
        self._lib.lunelette_metal_last_device_ms(self.handle, ctypes.byref(ms))
        return ms.value

    def read_kv(self, layer, kind, position, count):
        out = np.empty(count * 1024, np.float32)
        if self._lib.lunelette_metal_read_kv(self.handle, layer, kind, position, count,
                                             out.ctypes.data_as(c_float_p)):
            raise RuntimeError_("read_kv failed")
        return out.reshape(count, 1024)

    def inject(self, what):
        """Test build only: 1 fail before device work, 2 Inf logit, 3 checkpoint
        allocation failure, 6 the one-launch attention blocks give up, 7 the
        attention's flag combiners give up (next call)."""
        if self._lib.lunelette_metal_test_inject(self.handle, what):
            raise RuntimeError_("inject rejected")

    def fail_after_layer(self, layer):
        """Test build only: the next execution fails after `layer`'s kernels."""
        if self._lib.lunelette_metal_test_fail_after_layer(self.handle, layer):
            raise RuntimeError_("fail_after_layer rejected")

    def set_epoch(self, epoch):
        """Test build only: sets the checkpoint epoch counter."""
        if self._lib.lunelette_metal_test_set_epoch(self.handle, epoch):
            raise RuntimeError_("set_epoch rejected")

    def set_logit(self, index, value):
        """Test build only: overwrites one published host logit."""
        if self._lib.lunelette_metal_test_set_logit(self.handle, index, value):
            raise RuntimeError_("set_logit rejected")

    @property
    def last_error(self):
        return self._err.value.decode()
