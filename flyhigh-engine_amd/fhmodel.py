"""Python host driver of the model ABI of libfhconv.so (include/fhc_model.h): the FlyHighFG model files and the
static plan of a frame.

``Model.load(dir)`` reads graph.json, flyhighfg.json and flyhighfg.bin from a directory the caller names (the
reference's Model::from_dir, crates/flyhigh-engine/src/model/mod.rs:38-96); ``info()``, ``shape(name)`` and
``weight(name)`` (f16 bits, model/blob.rs:29-41) read it; ``plan(k, frame, network, repair)`` walks the graph into
the plan of one pair() + mid() (net/build.rs:149-736, net/session.rs:26-66); ``conv_shapes`` and ``autotune``
discover and tune its conv shapes (ops/conv/autotune.rs:153-245). Errors raise ``FhcError`` with the library's
message. No model file travels with this repository.
"""
from __future__ import annotations

import ctypes
import json
from typing import Optional, Tuple

import fhconv
from fhconv import FhcError

_typed = False


def _lib():
    global _typed
    L = fhconv.load()
    if not _typed:
        P, U32, SZ = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_size_t
        sig = {
            "fhc_model_load": ([ctypes.c_char_p, ctypes.POINTER(P)], ctypes.c_int),
            "fhc_model_load_bytes": ([ctypes.c_char_p, SZ, ctypes.c_char_p, SZ, P, SZ, ctypes.POINTER(P)],
                                     ctypes.c_int),
            "fhc_model_destroy": ([P], None),
            "fhc_model_info": ([P, ctypes.c_char_p, SZ], ctypes.c_int),
            "fhc_model_tensor": ([P, ctypes.c_char_p, ctypes.POINTER(U32), SZ, ctypes.POINTER(ctypes.c_uint64)],
                                 ctypes.c_int),
            "fhc_model_weight": ([P, ctypes.c_char_p, P, SZ], ctypes.c_int64),
            "fhc_model_plan": ([P, U32, U32, U32, U32, U32, U32, ctypes.c_char_p, SZ], ctypes.c_int),
            "fhc_model_conv_shapes": ([P, U32, U32, U32, U32, U32, U32, ctypes.POINTER(U32), SZ], ctypes.c_int),
            "fhc_model_autotune": ([P, U32, U32, U32, U32, U32, U32, ctypes.c_int], ctypes.c_int),
        }
        for name, (args, res) in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _typed = True
    return L


def _check(rc, what):
    if rc < 0:
        raise FhcError(f"{what}: {fhconv.last_error()}")
    return rc


class Model:
    def __init__(self, handle):
        self._h = handle

    @classmethod
    def load(cls, directory: str) -> "Model":
        h = ctypes.c_void_p()
        _check(_lib().fhc_model_load(directory.encode(), ctypes.byref(h)), "fhc_model_load")
        return cls(h)

    @classmethod
    def from_bytes(cls, graph_json: bytes, manifest_json: bytes, blob: bytes) -> "Model":
        h = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(blob, len(blob)) if blob else None
        _check(_lib().fhc_model_load_bytes(graph_json, len(graph_json), manifest_json, len(manifest_json),
                                           ctypes.cast(buf, ctypes.c_void_p) if buf is not None else None,
                                           len(blob), ctypes.byref(h)), "fhc_model_load_bytes")
        return cls(h)

    def info(self) -> dict:
        buf = ctypes.create_string_buffer(1024)
        _check(_lib().fhc_model_info(self._h, buf, len(buf)), "fhc_model_info")
        return json.loads(buf.value.decode())

    def shape(self, name: str) -> Optional[Tuple[int, ...]]:
        dims, count = (ctypes.c_uint32 * 8)(), ctypes.c_uint64()
        n = _lib().fhc_model_tensor(self._h, name.encode(), dims, 8, ctypes.byref(count))
        return None if n < 0 else tuple(dims[:n])

    def weight(self, name: str):
        """The tensor's f16 bit patterns (numpy uint16), in the blob's order (OIHW for a conv)."""
        import numpy as np
        shape = self.shape(name)
        if shape is None:
            raise FhcError(f"fhc_model_weight: no tensor {name}")
        out = np.empty(int(np.prod(shape)) if shape else 1, np.uint16)
        _check(_lib().fhc_model_weight(self._h, name.encode(), out.ctypes.data, out.size), "fhc_model_weight")
        return out.reshape(shape)

    def plan(self, k: int, frame: Tuple[int, int], network: Tuple[int, int], repair: int = 1) -> dict:
        """The static plan of one pair() + mid() for frames of frame = (w, h) at the network size (w, h), with the
        periodic-structure repair at level `repair` (0 off; 1, the reference's default)."""
        cap = 1 << 20
        while True:
            buf = ctypes.create_string_buffer(cap)
            rc = _lib().fhc_model_plan(self._h, k, frame[0], frame[1], network[0], network[1], repair, buf, cap)
            if rc >= 0:
                return json.loads(buf.value.decode())
            if "buffer too small" not in fhconv.last_error():
                _check(rc, "fhc_model_plan")
            cap *= 4

    def conv_shapes(self, k: int, frame: Tuple[int, int], network: Tuple[int, int], n: int = 1) -> list:
        """The plan's distinct conv shapes at batch n: (cin, cout, h, w, stride, n, kernel size), h, w the input."""
        cap = 7 * 256
        buf = (ctypes.c_uint32 * cap)()
        cnt = _check(_lib().fhc_model_conv_shapes(self._h, k, frame[0], frame[1], network[0], network[1], n, buf,
                                                   cap), "fhc_model_conv_shapes")
        return [tuple(buf[7 * i:7 * i + 7]) for i in range(min(cnt, cap // 7))]

    def autotune(self, k: int, frame: Tuple[int, int], network: Tuple[int, int], n: int = 1, reps: int = 10) -> int:
        """Tune every conv shape of the plan into the choice table (fhc_model_autotune); the number tuned."""
        return _check(_lib().fhc_model_autotune(self._h, k, frame[0], frame[1], network[0], network[1], n, reps),
                      "fhc_model_autotune")

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            _lib().fhc_model_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
