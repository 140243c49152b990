"""Python view of the native session adapter (include/lunelette_session.h).

The adapter is the service's model-facing state machine (chunked
materialization with the legacy/on/off prefix-reuse policies, checkpoint
save/restore, greedy or forced selection with the LNRPLY1 capture) over one
runtime context. Every call goes to the C library; this class only converts
arguments and results.
"""
import ctypes
import json

import numpy as np

from . import (COMPACT_FP8_ARITHMETIC, Options, PREFILL_MPS, SessionOptions, SessionWork, VOCAB,
               lib)

LEGACY, REUSE_ON, REUSE_OFF = 0, 1, 2
MORE = 2
EOS = 2


def _tokens(tokens):
    array = np.ascontiguousarray(tokens, dtype=np.uint32)
    return array, array.ctypes.data_as(ctypes.POINTER(ctypes.c_uint))


class Session:
    """One adapter instance. `library` is the loaded C library that holds the
    adapter (the product by default)."""

    def __init__(self, handle, library):
        self._lib = library
        self.handle = handle

    @classmethod
    def open(cls, model, context=4352, block=256, prefix_reuse=LEGACY, prefill=PREFILL_MPS,
             strategy=COMPACT_FP8_ARITHMETIC, replay_path=None, library=None):
        """lunelette_session_open: loads the checkpoint file `model`."""
        library = library or lib()
        err = ctypes.create_string_buffer(512)
        opts = SessionOptions(context, block, prefix_reuse,
                              replay_path.encode() if replay_path else None)
        handle = library.lunelette_session_open(str(model).encode(),
                                                ctypes.byref(Options(prefill, strategy)),
                                                ctypes.byref(opts), err, 512)
        if not handle:
            raise RuntimeError("session open failed: " + err.value.decode())
        return cls(handle, library)

    @classmethod
    def adopt(cls, runtime, prefix_reuse=LEGACY, replay_path=None, library=None):
        """lunelette_session_adopt over a runtime.Runtime, with the options and
        limits it was created with; the session takes ownership of the
        context in every case."""
        library = library or lib()
        handle, runtime.handle = runtime.handle, None
        err = ctypes.create_string_buffer(512)
        opts = SessionOptions(runtime.context, runtime.block, prefix_reuse,
                              replay_path.encode() if replay_path else None)
        created = Options(runtime.prefill_mode, runtime.strategy)
        session = library.lunelette_session_adopt(handle, ctypes.byref(created),
                                                  ctypes.byref(opts), err, 512)
        if not session:
            raise RuntimeError("session adopt failed: " + err.value.decode())
        return cls(session, library)

    def close(self):
        if self.handle:
            self._lib.lunelette_session_destroy(self.handle)
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

    def materialize(self, tokens):
        """0 rejected/failed, 1 ready, MORE one block committed."""
        array, ptr = _tokens(tokens)
        return self._lib.lunelette_session_materialize(self.handle, ptr, array.size)

    def materialize_step(self, tokens):
        """(result, committed length)."""
        array, ptr = _tokens(tokens)
        cursor = ctypes.c_uint(0)
        result = self._lib.lunelette_session_materialize_step(self.handle, ptr, array.size,
                                                              ctypes.byref(cursor))
        return result, cursor.value

    def ingest(self, tokens):
        """materialize_step until READY; returns (result, [receipts])."""
        receipts = []
        while True:
            result, _ = self.materialize_step(tokens)
            receipts.append(self.work())
            if result != MORE:
                return result, receipts

    def next(self):
        return self._lib.lunelette_session_next(self.handle)

    def replay_next(self, forced):
        return self._lib.lunelette_session_replay_next(self.handle, forced)

    def save(self):
        return self._lib.lunelette_session_save(self.handle)

    def restore(self):
        return self._lib.lunelette_session_restore(self.handle)

    def begin(self):
        self._lib.lunelette_session_begin(self.handle)

    def invalidate(self):
        self._lib.lunelette_session_invalidate(self.handle)

    def reset(self):
        self._lib.lunelette_session_reset(self.handle)

    def work(self):
        """Takes the receipt of the last materialize/restore as a dict."""
        w = SessionWork()
        self._lib.lunelette_session_take_work(self.handle, ctypes.byref(w))
        return {name: getattr(w, name) for name, _ in SessionWork._fields_}

    def logits(self):
        """Copy of the current logits, or None when they are stale."""
        ptr = self._lib.lunelette_session_logits(self.handle)
        if not ptr:
            return None
        return np.ctypeslib.as_array(ptr, shape=(VOCAB,)).copy()

    @property
    def length(self):
        return self._lib.lunelette_session_length(self.handle)

    @property
    def context_capacity(self):
        return self._lib.lunelette_session_context_capacity(self.handle)

    @property
    def block_capacity(self):
        return self._lib.lunelette_session_block_capacity(self.handle)

    @property
    def prefix_reuse(self):
        return self._lib.lunelette_session_prefix_reuse(self.handle)

    @property
    def error(self):
        return self._lib.lunelette_session_error(self.handle).decode()

    @property
    def info_text(self):
        return self._lib.lunelette_session_info(self.handle).decode()

    @property
    def info(self):
        return json.loads(self.info_text)
