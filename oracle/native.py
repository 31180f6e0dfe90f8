"""ctypes wrappers over the CPU checkers built by oracle/Makefile. TEST INFRASTRUCTURE ONLY.

* `OracleGemm`  this repo's C restatement (`_build/libmx_oracle.so`).
* `RefGemm`     the reference's own C kernels compiled from /root/reference
                (`_ref/libmx_ref.so`, or `_ref/libmx_ref_nofma.so` with contraction off): the
                functions bound are the reference's `mx_gemm` (app/native/src/mx_gemm.c:125),
                `mx_supports` (:209), `mx_quantize_row_q8_k` (mx_common.c:42) and
                `mx_dequant_rows` (mx_dequant_rows.c:77), with the argument types the
                reference's own binding declares (app/native/gemm.py:31-61).
"""

import ctypes
import os
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
ORACLE_LIB = ORACLE_DIR / "_build" / "libmx_oracle.so"
REF_LIB = ORACLE_DIR / "_ref" / "libmx_ref.so"
REF_LIB_NOFMA = ORACLE_DIR / "_ref" / "libmx_ref_nofma.so"

_vp = ctypes.c_void_p
_i = ctypes.c_int


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def default_threads() -> int:
    """Host threads for the CPU paths: the OpenMP setting if given, else the CPUs this process
    may run on."""
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


class OracleGemm:
    def __init__(self, path: Path = ORACLE_LIB) -> None:
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built (run `make -C oracle`)")
        lib = ctypes.CDLL(str(path))
        lib.mxo_gemm.argtypes = [_i, _vp, _vp, _vp, _i, _i, _i, _i]
        lib.mxo_gemm.restype = _i
        lib.mxo_supports.argtypes = [_i, _i]
        lib.mxo_supports.restype = _i
        lib.mxo_quantize_q8_k.argtypes = [_vp, _vp, _vp, _vp, _i, _i]
        lib.mxo_quantize_q8_k.restype = None
        lib.mxo_dequantize.argtypes = [_i, _vp, ctypes.c_long, _vp]
        lib.mxo_dequantize.restype = _i
        self._lib = lib

    def supports(self, ggml_type: int, in_features: int) -> bool:
        return bool(self._lib.mxo_supports(ggml_type, in_features))

    def gemm(self, ggml_type: int, packed: np.ndarray, x: np.ndarray, out_features: int,
             in_features: int, n_threads: int | None = None) -> np.ndarray:
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_features)
        y = np.empty((x.shape[0], out_features), dtype=np.float32)
        status = self._lib.mxo_gemm(ggml_type, _ptr(packed), _ptr(x), _ptr(y), x.shape[0],
                                    out_features, in_features, n_threads or default_threads())
        if status != 0:
            raise RuntimeError(f"mxo_gemm failed with status {status}")
        return y

    def quantize_q8_k(self, x: np.ndarray):
        x = np.ascontiguousarray(x, dtype=np.float32)
        m, k = x.shape
        q = np.empty((m, k), dtype=np.int8)
        d = np.empty((m, k // 256), dtype=np.float32)
        bs = np.empty((m, k // 256, 16), dtype=np.int16)
        self._lib.mxo_quantize_q8_k(_ptr(x), _ptr(q), _ptr(d), _ptr(bs), m, k)
        return q, d, bs

    def dequantize(self, ggml_type: int, blocks: np.ndarray, n_blocks: int) -> np.ndarray:
        from oracle.dequant import GEOMETRY

        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        out = np.empty(n_blocks * GEOMETRY[ggml_type][0], dtype=np.float32)
        if self._lib.mxo_dequantize(ggml_type, _ptr(blocks), n_blocks, _ptr(out)) != 0:
            raise RuntimeError("mxo_dequantize: unsupported type")
        return out


class _Q8KBlock(ctypes.Structure):
    """The reference's activation block `mx_block_q8_k` (app/native/src/mx_common.h:68-72)."""

    _fields_ = [("d", ctypes.c_float), ("qs", ctypes.c_int8 * 256), ("bsums", ctypes.c_int16 * 16)]


class RefGemm:
    """The reference C kernels (built from /root/reference by oracle/Makefile)."""

    def __init__(self, path: Path = REF_LIB) -> None:
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built (run `make -C oracle ref`)")
        os.environ.setdefault("OMP_WAIT_POLICY", "PASSIVE")  # as app/native/library.py:102
        lib = ctypes.CDLL(str(path))
        lib.mx_gemm.argtypes = [_i, _vp, _vp, _vp, _i, _i, _i, _i]
        lib.mx_gemm.restype = _i
        lib.mx_supports.argtypes = [_i, _i]
        lib.mx_supports.restype = _i
        lib.mx_quantize_row_q8_k.argtypes = [_vp, _vp, _i]
        lib.mx_quantize_row_q8_k.restype = None
        lib.mx_dequant_rows.argtypes = [_i, _vp, _vp, _i, _i, _vp, _i]
        lib.mx_dequant_rows.restype = _i
        lib.mx_build_info.restype = ctypes.c_char_p
        lib.mx_rms_norm.argtypes = [_vp, _vp, _vp, _i, _i, ctypes.c_float]
        lib.mx_rms_norm.restype = None
        lib.mx_silu_mul.argtypes = [_vp, _vp, _vp, _i]
        lib.mx_silu_mul.restype = None
        self._lib = lib
        self.build_info = lib.mx_build_info().decode()

    def supports(self, ggml_type: int, in_features: int) -> bool:
        return bool(self._lib.mx_supports(ggml_type, in_features))

    def gemm(self, ggml_type: int, packed: np.ndarray, x: np.ndarray, out_features: int,
             in_features: int, n_threads: int | None = None) -> np.ndarray:
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_features)
        y = np.empty((x.shape[0], out_features), dtype=np.float32)
        status = self._lib.mx_gemm(ggml_type, _ptr(packed), _ptr(x), _ptr(y), x.shape[0],
                                   out_features, in_features, n_threads or default_threads())
        if status != 0:
            raise RuntimeError(f"mx_gemm failed with status {status}")
        return y

    def quantize_q8_k(self, x: np.ndarray):
        """(q int8 (M,K), d float32 (M,K/256), bsums int16 (M,K/256,16)) via the reference."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        m, k = x.shape
        nb = k // 256
        q = np.empty((m, k), dtype=np.int8)
        d = np.empty((m, nb), dtype=np.float32)
        bs = np.empty((m, nb, 16), dtype=np.int16)
        for r in range(m):
            blocks = (_Q8KBlock * nb)()
            self._lib.mx_quantize_row_q8_k(_ptr(x[r]), ctypes.addressof(blocks), k)
            for b in range(nb):
                q[r, b * 256 : (b + 1) * 256] = np.frombuffer(blocks[b].qs, dtype=np.int8)
                d[r, b] = blocks[b].d
                bs[r, b] = np.frombuffer(blocks[b].bsums, dtype=np.int16)
        return q, d, bs

    def dequant_rows(self, ggml_type: int, packed: np.ndarray, rows: np.ndarray,
                     row_width: int) -> np.ndarray:
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        rows = np.ascontiguousarray(rows, dtype=np.int32)
        out = np.empty((rows.shape[0], row_width), dtype=np.float32)
        status = self._lib.mx_dequant_rows(ggml_type, _ptr(packed), _ptr(rows), rows.shape[0],
                                           row_width, _ptr(out), 1)
        if status != 0:
            raise RuntimeError(f"mx_dequant_rows failed with status {status}")
        return out


    def rms_norm(self, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty_like(x)
        self._lib.mx_rms_norm(_ptr(x), _ptr(w), _ptr(out), x.shape[0], x.shape[1], float(eps))
        return out

    def silu_mul(self, gate: np.ndarray, up: np.ndarray) -> np.ndarray:
        g = np.ascontiguousarray(gate, dtype=np.float32)
        u = np.ascontiguousarray(up, dtype=np.float32)
        out = np.empty_like(g)
        self._lib.mx_silu_mul(_ptr(g), _ptr(u), _ptr(out), g.size)
        return out


def ref_available(nofma: bool = False) -> bool:
    return (REF_LIB_NOFMA if nofma else REF_LIB).exists()
