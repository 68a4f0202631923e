"""ctypes binding of the C oracle restatement (vq_oracle.c) -- test
infrastructure only. Builds libvqoracle.so with `make` when it is absent."""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "libvqoracle.so"


def build(force: bool = False) -> pathlib.Path:
    if force or not LIB.exists():
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=HERE, check=True)
    return LIB


class COracle:
    def __init__(self, path):
        self.lib = ctypes.CDLL(str(path))
        L = self.lib
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.vqo_pack.argtypes = [P, P, I64, I, I]
        L.vqo_unpack.argtypes = [P, P, I64, I, I]
        L.vqo_f32_to_f16.argtypes = [ctypes.c_float]
        L.vqo_f32_to_f16.restype = ctypes.c_uint16
        L.vqo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.vqo_f16_to_f32.restype = ctypes.c_float
        L.vqo_dequant.argtypes = [P, P, I, P, I, I64, I, P]
        L.vqo_gemv_f32.argtypes = [P, P, I64, I64, I64, P]
        L.vqo_f32_to_f16_array.argtypes = [P, P, I64]

    @staticmethod
    def _p(a):
        return a.ctypes.data_as(ctypes.c_void_p)

    def pack(self, codes, bits):
        codes = np.ascontiguousarray(codes, np.uint16)
        lead, nsub = codes.shape[:-1], codes.shape[-1]
        wpr = (nsub + 31) // 32 * bits
        out = np.zeros(lead + (wpr,), np.uint32)
        rc = self.lib.vqo_pack(self._p(codes), self._p(out), int(np.prod(lead, dtype=np.int64)), nsub, bits)
        if rc:
            raise ValueError(f"vqo_pack rc={rc}")
        return out

    def unpack(self, packed, nsub, bits):
        packed = np.ascontiguousarray(packed, np.uint32)
        lead = packed.shape[:-1]
        out = np.zeros(lead + (nsub,), np.uint16)
        rc = self.lib.vqo_unpack(self._p(packed), self._p(out), int(np.prod(lead, dtype=np.int64)), nsub, bits)
        if rc:
            raise ValueError(f"vqo_unpack rc={rc}")
        return out

    def f32_to_f16_bits(self, values):
        v = np.ascontiguousarray(values, np.float32).reshape(-1)
        out = np.zeros(v.shape, np.uint16)
        self.lib.vqo_f32_to_f16_array(self._p(v), self._p(out), v.size)
        return out

    def dequant(self, codes, codebook, scales, group):
        codes = np.ascontiguousarray(codes, np.uint16)
        cb = np.ascontiguousarray(codebook, np.float16).view(np.uint16)
        sc = np.ascontiguousarray(scales, np.float16).view(np.uint16)
        lead, nsub = codes.shape[:-1], codes.shape[-1]
        d = cb.shape[1]
        out = np.zeros(lead + (nsub * d,), np.uint16)
        self.lib.vqo_dequant(self._p(codes), self._p(cb), d, self._p(sc), group,
                             int(np.prod(lead, dtype=np.int64)), nsub, self._p(out))
        return out.view(np.float16)

    def gemv_f32(self, x, w16):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w16, np.float16).view(np.uint16)
        y = np.zeros((x.shape[0], w.shape[0]), np.float32)
        self.lib.vqo_gemv_f32(self._p(x), self._p(w), x.shape[0], w.shape[0], x.shape[1], self._p(y))
        return y


def load() -> COracle:
    return COracle(build())
