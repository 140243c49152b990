"""Python view of the Tekken tokenizer and chat framing
(include/lunelette_tokenizer.h, include/lunelette_chat.h).

`library` selects the C library holding the functions: the product by
default, or any library with the same entry points (the tests load the
reference's tokenizer built from source through the same class)."""
import ctypes

import numpy as np

from . import c_int64_p, lib

MAX_INPUT = 4096
LONG_INPUT = 32768


class Tokenizer:
    def __init__(self, path, library=None):
        self._lib = library or lib()
        handle = ctypes.c_void_p()
        err = ctypes.create_string_buffer(512)
        if not self._lib.lunelette_tokenizer_open(str(path).encode(), ctypes.byref(handle), err,
                                                  512):
            raise ValueError(err.value.decode())
        self.handle = handle.value

    def close(self):
        if self.handle:
            self._lib.lunelette_tokenizer_close(self.handle)
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

    def encode(self, text, limit=None):
        """Ids of `text` (bytes or str); ValueError with the diagnostic."""
        data = text.encode() if isinstance(text, str) else bytes(text)
        ids = ctypes.POINTER(ctypes.c_uint32)()
        count = ctypes.c_size_t()
        err = ctypes.create_string_buffer(512)
        if limit is None:
            ok = self._lib.lunelette_tokenizer_encode(self.handle, data, len(data),
                                                      ctypes.byref(ids), ctypes.byref(count),
                                                      err, 512)
        else:
            ok = self._lib.lunelette_tokenizer_encode_with_limit(self.handle, data, len(data),
                                                                 limit, ctypes.byref(ids),
                                                                 ctypes.byref(count), err, 512)
        if not ok:
            assert not ids and count.value == 0
            raise ValueError(err.value.decode())
        out = [ids[i] for i in range(count.value)]
        _free(ids)
        return out

    def decode(self, ids):
        array = (ctypes.c_uint32 * max(len(ids), 1))(*ids)
        data = ctypes.POINTER(ctypes.c_ubyte)()
        length = ctypes.c_size_t()
        err = ctypes.create_string_buffer(512)
        if not self._lib.lunelette_tokenizer_decode(self.handle, array if ids else None, len(ids),
                                                    ctypes.byref(data), ctypes.byref(length),
                                                    err, 512):
            assert not data and length.value == 0
            raise ValueError(err.value.decode())
        out = ctypes.string_at(data, length.value)
        _free(data)
        return out

    def chat_prompt(self, prompt, system=None, raw=False):
        """(status, ids) of lunelette_chat_prompt."""
        ids = np.full(256, -7, np.int64)
        count = ctypes.c_size_t(999)
        err = ctypes.create_string_buffer(512)
        status = self._lib.lunelette_chat_prompt(
            self.handle, prompt.encode() if isinstance(prompt, str) else prompt,
            None if system is None else (system.encode() if isinstance(system, str) else system),
            int(raw), ids.ctypes.data_as(c_int64_p), ctypes.byref(count), err, 512)
        return status, ids[:count.value].tolist() if status == 0 else None


_libc = ctypes.CDLL(None)
_libc.free.argtypes = [ctypes.c_void_p]


def _free(pointer):
    _libc.free(ctypes.cast(pointer, ctypes.c_void_p))


def split(text, library=None):
    """Byte offsets where the pre-tokenizer's pieces end."""
    data = text.encode() if isinstance(text, str) else bytes(text)
    ends = (ctypes.c_size_t * max(len(data), 1))()
    n = (library or lib()).lunelette_tokenizer_split(data, len(data), ends, len(ends))
    if n < 0:
        raise ValueError("invalid UTF-8 or input")
    return [ends[i] for i in range(n)]
