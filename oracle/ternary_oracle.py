"""CPU oracle for the ternary linear layer (numpy side).  TEST INFRASTRUCTURE ONLY.

Only the tests, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` import this module, and only as the checker.  The product path
never imports, links or calls anything under ``oracle/``.

It holds:

* closed forms pinned by the mathematics (reference paths relative to
  ``src/ivonar_inference/``):
  - ``pack_codes`` / ``unpack_codes``: quantization.py:13-18 (byte b holds
    inputs 4b+k in bits 2k..2k+1, code = w + 1), tests/conftest.py:55-61;
  - ``quantize_closed_form``: quantization.py:35-38 and ternary.cu:178-186,
    amax -> s = max(amax/127, 1e-5) in IEEE fp32 -> q = round-half-even(x/s);
  - ``group_partials_int64``: brute-force per-128-group sums of (code-1)*q;
  - ``truth_fp64``: s_x * sum_g P[r,g] * scale[r,g] + b in float64;
* ctypes bindings of ``liboracle.so`` (oracle.c), which restates the same
  semantics in the exact fp32 orders of the HIP kernels and of the reference
  kernel, and of ``libcpubaseline.so`` (the numba kernels restated in C++).
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_int64, c_uint16, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
GROUP = 128
CHUNK = 64
MODE_PLAIN, MODE_NORM, MODE_ATTN = 0, 1, 2
EPI_STORE, EPI_RESIDUAL, EPI_SILU_PAIR = 0, 1, 2


# --------------------------------------------------------------------------- closed forms


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """codes uint8 [N, K] in {0,1,2} -> packed uint8 [N, ceil(K/4)] (quantization.py:13-18 inverse)."""
    codes = np.asarray(codes, dtype=np.uint8)
    n_rows, k = codes.shape
    width = math.ceil(k / 4)
    padded = np.zeros((n_rows, width * 4), dtype=np.uint8)
    padded[:, :k] = codes
    quads = padded.reshape(n_rows, width, 4)
    return (quads[..., 0] | (quads[..., 1] << 2) | (quads[..., 2] << 4) | (quads[..., 3] << 6)).astype(np.uint8)


def unpack_codes(packed: np.ndarray, k: int) -> np.ndarray:
    """packed uint8 [N, W] -> codes uint8 [N, k] (quantization.py:13-18, before the -1)."""
    packed = np.asarray(packed, dtype=np.uint8)
    values = np.stack([packed & 3, (packed >> 2) & 3, (packed >> 4) & 3, (packed >> 6) & 3], axis=-1)
    return values.reshape(packed.shape[0], -1)[:, :k]


def pad_rows16(packed: np.ndarray) -> np.ndarray:
    """Pad each packed row with zero bytes to a multiple of 16 (kernel_decoder.py:107-110)."""
    rows, width = packed.shape
    padded = (width + 15) // 16 * 16
    out = np.zeros((rows, padded), dtype=np.uint8)
    out[:, :width] = packed
    return out


def quantize_closed_form(x: np.ndarray) -> tuple[np.ndarray, np.float32]:
    """Plain per-token quantizer in IEEE fp32: returns (q int64 [K] in input order, scale)."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.float32(np.max(np.abs(x))) if x.size else np.float32(0.0)
    scale = np.maximum(np.float32(amax / np.float32(127.0)), np.float32(1e-5)).astype(np.float32)
    q = np.rint(x / scale).astype(np.int64)
    return q, np.float32(scale)


def q8_index(n: int) -> np.ndarray:
    """Byte offset of each input in the q8 layout (same as oracle.c q8_index)."""
    i = np.arange(n)
    return (i >> 6) * 64 + ((i >> 4) & 3) * 16 + (i & 3) * 4 + ((i >> 2) & 3)


def q8_linear(q8: np.ndarray, n: int) -> np.ndarray:
    """Inverse of the q8 layout: int8 activations in input order [..., n]."""
    return np.ascontiguousarray(np.asarray(q8)[..., q8_index(n)])


def q8_layout(q: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Linear-order int q [K] -> (q8 int8 [C*64] in the q8 layout, xsum int32 [C])."""
    n = q.shape[-1]
    chunks = (n + 63) // 64
    q8 = np.zeros(chunks * 64, dtype=np.int8)
    q8[q8_index(n)] = q.astype(np.int8)
    padded = np.zeros(chunks * 64, dtype=np.int64)
    padded[:n] = q
    return q8, padded.reshape(chunks, 64).sum(-1).astype(np.int32)


def group_partials_int64(codes: np.ndarray, q: np.ndarray) -> np.ndarray:
    """Brute force P[r, g] = sum_{i in g} (code - 1) * q, int64."""
    rows, k = codes.shape
    groups = (k + GROUP - 1) // GROUP
    w = np.zeros((rows, groups * GROUP), dtype=np.int64)
    w[:, :k] = codes.astype(np.int64) - 1
    qp = np.zeros(groups * GROUP, dtype=np.int64)
    qp[:k] = q
    return (w.reshape(rows, groups, GROUP) * qp.reshape(groups, GROUP)).sum(-1)


def half_bits_to_float(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def truth_fp64(partials: np.ndarray, scales_f32: np.ndarray, sx: float, bias: np.ndarray | None = None) -> np.ndarray:
    """fp64 output: sx * sum_g P[r,g] * scale[r,g] (+ bias)."""
    y = (partials.astype(np.float64) * scales_f32.astype(np.float64)).sum(-1) * float(sx)
    if bias is not None:
        y = y + bias.astype(np.float64)
    return y


def within(actual: np.ndarray, expected: np.ndarray, rtol: float = 1e-5, atol: float = 1e-6) -> np.ndarray:
    """Element-wise |actual - expected| <= atol + rtol * |expected|."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    return np.abs(actual - expected) <= atol + rtol * np.abs(expected)


# --------------------------------------------------------------------------- C oracle


def build() -> None:
    """Compile liboracle.so and libcpubaseline.so with oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def _load(name: str) -> ctypes.CDLL:
    path = HERE / name
    if not path.is_file():
        build()
    return ctypes.CDLL(str(path))


def _ptr(array: np.ndarray | None) -> c_void_p:
    if array is None:
        return c_void_p(0)
    if not array.flags["C_CONTIGUOUS"]:
        raise ValueError("oracle arrays must be C-contiguous")
    return c_void_p(array.ctypes.data)


class Oracle:
    """ctypes view of liboracle.so; every array argument is a numpy array."""

    def __init__(self) -> None:
        lib = _load("liboracle.so")
        lib.orc_h2f.argtypes = [c_uint16]
        lib.orc_h2f.restype = c_float
        lib.orc_expf.argtypes = [c_float]
        lib.orc_expf.restype = c_float
        lib.orc_silu.argtypes = [c_float]
        lib.orc_silu.restype = c_float
        lib.orc_ref_sum_squares.argtypes = [c_void_p, c_int]
        lib.orc_ref_sum_squares.restype = c_float
        lib.orc_quantize_rows.argtypes = [c_int, c_void_p, c_int, c_void_p, c_int, c_float, c_int, c_int, c_int,
                                          c_void_p, c_void_p, c_void_p]
        lib.orc_group_partials.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]
        lib.orc_gemv_pairs.argtypes = [c_int, c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_int, c_int, c_int, c_int, c_int]
        lib.orc_gemm_seq.argtypes = [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                     c_int, c_int, c_int, c_int, c_int, c_int]
        lib.orc_gemm_split.argtypes = [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_int, c_int, c_int, c_int, c_int, c_int, c_int]
        lib.orc_reforder.argtypes = [c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int]
        lib.orc_embed.argtypes = [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int]
        lib.orc_partials_i8.argtypes = [c_void_p, c_int, c_int, c_void_p, c_void_p]
        lib.orc_finish.argtypes = [c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                   c_int, c_int, c_int, c_int]
        lib.orc_argmax.argtypes = [c_void_p, c_int]
        lib.orc_argmax.restype = c_int64
        lib.orc_logit_bounds.argtypes = [c_void_p, c_float, c_float, c_float, c_void_p, c_void_p, c_int]
        lib.orc_sample_token.argtypes = [c_void_p, c_float, c_float, c_float, c_void_p, c_int64, c_int, c_float, c_int,
                                         c_void_p, c_void_p, c_void_p]
        lib.orc_sample_token.restype = c_int64
        self.lib = lib

    def expf(self, x: float) -> float:
        return float(self.lib.orc_expf(float(x)))

    def expf_array(self, x: np.ndarray) -> np.ndarray:
        return np.array([self.lib.orc_expf(float(v)) for v in np.asarray(x, dtype=np.float32)], dtype=np.float32)

    def silu_array(self, x: np.ndarray) -> np.ndarray:
        return np.array([self.lib.orc_silu(float(v)) for v in np.asarray(x, dtype=np.float32)], dtype=np.float32)

    def h2f(self, bits: int) -> float:
        return float(self.lib.orc_h2f(int(bits)))

    def ref_sum_squares(self, v: np.ndarray) -> np.float32:
        v = np.ascontiguousarray(v, dtype=np.float32)
        return np.float32(self.lib.orc_ref_sum_squares(_ptr(v), v.shape[0]))

    def quantize_rows(self, mode: int, x: np.ndarray, n: int, aux: np.ndarray | None = None, eps: float = 1e-6,
                      splits: int = 1, head_dim: int = 64, m: int | None = None, in_stride: int | None = None):
        """Returns (q8 int8 [m, C*64], xsum int32 [m, C], scale fp32 [m])."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if m is None:
            m = 1 if x.ndim == 1 else x.shape[0]
        if in_stride is None:
            in_stride = x.shape[-1] if x.ndim > 1 else n
        chunks = (n + 63) // 64
        q8 = np.zeros((m, chunks * 64), dtype=np.int8)
        xsum = np.zeros((m, chunks), dtype=np.int32)
        scale = np.zeros(m, dtype=np.float32)
        aux_arr = None if aux is None else np.ascontiguousarray(aux, dtype=np.float32)
        self.lib.orc_quantize_rows(mode, _ptr(x), in_stride, _ptr(aux_arr), n, eps, splits, head_dim, m,
                                   _ptr(q8), _ptr(xsum), _ptr(scale))
        return q8, xsum, scale

    def group_partials(self, q8: np.ndarray, xsum: np.ndarray, packed: np.ndarray, rows: int, n: int) -> np.ndarray:
        groups = (n + 127) // 128
        out = np.zeros((rows, groups), dtype=np.int32)
        packed = np.ascontiguousarray(packed)
        self.lib.orc_group_partials(_ptr(np.ascontiguousarray(q8)), _ptr(np.ascontiguousarray(xsum)), _ptr(packed),
                                    rows, n, packed.shape[1], _ptr(out))
        return out

    def gemv_pairs(self, epi: int, q8, xsum, sx: float, packed, scales_bits, bias, out: np.ndarray, n: int,
                   lanes: int) -> np.ndarray:
        packed = np.ascontiguousarray(packed)
        scales_bits = np.ascontiguousarray(scales_bits, dtype=np.uint16)
        self.lib.orc_gemv_pairs(epi, _ptr(np.ascontiguousarray(q8)), _ptr(np.ascontiguousarray(xsum)), float(sx),
                                _ptr(packed), _ptr(scales_bits), _ptr(bias), _ptr(out), packed.shape[0], n,
                                packed.shape[1], scales_bits.shape[1], lanes)
        return out

    def gemm_seq(self, epi: int, q8, xsum, scale_in, packed, scales_bits, bias, out: np.ndarray, n: int,
                 out_stride: int, m: int) -> np.ndarray:
        packed = np.ascontiguousarray(packed)
        scales_bits = np.ascontiguousarray(scales_bits, dtype=np.uint16)
        self.lib.orc_gemm_seq(epi, _ptr(np.ascontiguousarray(q8)), _ptr(np.ascontiguousarray(xsum)),
                              _ptr(np.ascontiguousarray(scale_in, dtype=np.float32)), _ptr(packed), _ptr(scales_bits),
                              _ptr(bias), _ptr(out), packed.shape[0], n, packed.shape[1], scales_bits.shape[1],
                              out_stride, m)
        return out

    def gemm_split(self, epi: int, q8, xsum, scale_in, packed, scales_bits, bias, out: np.ndarray, n: int,
                   out_stride: int, m: int, splits: int) -> np.ndarray:
        if splits < 1:
            raise ValueError(f"a K-split order needs at least one split, not {splits}")
        packed = np.ascontiguousarray(packed)
        scales_bits = np.ascontiguousarray(scales_bits, dtype=np.uint16)
        self.lib.orc_gemm_split(epi, _ptr(np.ascontiguousarray(q8)), _ptr(np.ascontiguousarray(xsum)),
                                _ptr(np.ascontiguousarray(scale_in, dtype=np.float32)), _ptr(packed), _ptr(scales_bits),
                                _ptr(bias), _ptr(out), packed.shape[0], n, packed.shape[1], scales_bits.shape[1],
                                out_stride, m, splits)
        return out

    def reforder(self, epi: int, tile: bool, q8, xsum, scale_in, packed, scales_bits, bias, out: np.ndarray, n: int,
                 lanes: int, out_stride: int, m: int) -> np.ndarray:
        packed = np.ascontiguousarray(packed)
        scales_bits = np.ascontiguousarray(scales_bits, dtype=np.uint16)
        self.lib.orc_reforder(epi, int(tile), _ptr(np.ascontiguousarray(q8)), _ptr(np.ascontiguousarray(xsum)),
                              _ptr(np.ascontiguousarray(scale_in, dtype=np.float32)), _ptr(packed), _ptr(scales_bits),
                              _ptr(bias), _ptr(out), packed.shape[0], n, packed.shape[1], scales_bits.shape[1],
                              lanes, out_stride, m)
        return out

    def partials_i8(self, w: np.ndarray, q_lin: np.ndarray) -> np.ndarray:
        """Exact int32 partials [rows, G] of int8 ternary values w [rows, K] against q [K] (input order)."""
        w = np.ascontiguousarray(w, dtype=np.int8)
        q_lin = np.ascontiguousarray(q_lin, dtype=np.int8)
        rows, k = w.shape
        out = np.zeros((rows, (k + 127) // 128), dtype=np.int32)
        self.lib.orc_partials_i8(_ptr(w), rows, k, _ptr(q_lin), _ptr(out))
        return out

    def finish(self, order: int, param: int, epi: int, partials: np.ndarray, scales_bits: np.ndarray, scale_in,
               bias, out: np.ndarray, k: int, out_stride: int) -> np.ndarray:
        """fp32 outputs from partials [m, rows, G]: order 0 = GEMV pairs (param = lanes), 1 = GEMM split."""
        if order not in (0, 1) or param < 1:
            raise ValueError(f"no fp32 order {order} with parameter {param}")
        partials = np.ascontiguousarray(partials, dtype=np.int32)
        if partials.ndim == 2:
            partials = partials[None]
        m, rows, _ = partials.shape
        scales_bits = np.ascontiguousarray(scales_bits, dtype=np.uint16)
        self.lib.orc_finish(order, param, epi, _ptr(partials), _ptr(scales_bits), scales_bits.shape[1],
                            _ptr(np.ascontiguousarray(scale_in, dtype=np.float32)), _ptr(bias), _ptr(out), rows, k,
                            out_stride, m)
        return out

    def embed(self, tokens: np.ndarray, packed, scales_bits, n: int) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, dtype=np.int64)
        packed = np.ascontiguousarray(packed)
        scales_bits = np.ascontiguousarray(scales_bits, dtype=np.uint16)
        out = np.zeros((tokens.shape[0], n), dtype=np.float32)
        self.lib.orc_embed(_ptr(tokens), tokens.shape[0], _ptr(packed), _ptr(scales_bits), _ptr(out), n,
                           packed.shape[1], scales_bits.shape[1])
        return out

    def argmax(self, x: np.ndarray) -> int:
        x = np.ascontiguousarray(x, dtype=np.float32)
        return int(self.lib.orc_argmax(_ptr(x), x.shape[0]))

    def logit_bounds(self, logits: np.ndarray, seen: np.ndarray, temperature: float, penalty: float,
                     inverse_penalty: float) -> np.ndarray:
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        seen = np.ascontiguousarray(seen, dtype=np.uint8)
        bounds = np.zeros((logits.shape[0] + 63) // 64, dtype=np.float32)
        self.lib.orc_logit_bounds(_ptr(logits), temperature, penalty, inverse_penalty, _ptr(seen), _ptr(bounds),
                                  logits.shape[0])
        return bounds

    def sample_token(self, logits: np.ndarray, seen: np.ndarray, temperature: float, penalty: float,
                     inverse_penalty: float, top_k: int, max_topk: int, uniform: float):
        """(token, picks in index order, their CDF); `seen` (uint8 numpy) gets seen[token] = 1."""
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        if seen.dtype != np.uint8 or not seen.flags.c_contiguous:
            raise TypeError("seen must be a contiguous uint8 array (it is updated in place)")
        picks = np.zeros(1024, dtype=np.int32)
        cdf = np.zeros(1024, dtype=np.float32)
        count = ctypes.c_int(0)
        token = self.lib.orc_sample_token(_ptr(logits), temperature, penalty, inverse_penalty, _ptr(seen), int(top_k),
                                          int(max_topk), uniform, logits.shape[0], _ptr(picks), _ptr(cdf),
                                          ctypes.byref(count))
        return int(token), picks[:count.value].copy(), cdf[:count.value].copy()


class CpuBaseline:
    """ctypes view of libcpubaseline.so (the numba kernels restated with OpenMP).  With ``native`` the
    library is rebuilt on this host with -march=native (libcpubaseline_native.so, make target ``native``);
    if that build fails the portable x86-64-v3 library is used and ``march`` says so."""

    def __init__(self, native: bool = False) -> None:
        self.march = "x86-64-v3"
        lib = None
        if native:
            done = subprocess.run(["make", "-s", "-B", "-C", str(HERE), "native"], capture_output=True, text=True)
            if done.returncode == 0:
                lib = ctypes.CDLL(str(HERE / "libcpubaseline_native.so"))
                self.march = "native"
            else:
                self.march = f"x86-64-v3 (native build failed: {done.stderr.strip()[-200:]})"
        if lib is None:
            lib = _load("libcpubaseline.so")
        lib.cb_planes_of.argtypes = [c_void_p, c_int, c_int, c_int, c_void_p]
        lib.cb_set_threads.argtypes = [c_int]
        lib.cb_max_threads.restype = c_int
        lib.cb_gemv.argtypes = [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                c_int]
        lib.cb_normed_gemv.argtypes = [c_void_p, c_void_p, c_float, c_float, c_int, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_int, c_void_p, c_void_p, c_void_p]
        lib.cb_normed_gemv_silu.argtypes = [c_void_p, c_void_p, c_float, c_float, c_int, c_void_p, c_void_p,
                                            c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p]
        self.lib = lib

    def set_threads(self, threads: int) -> None:
        self.lib.cb_set_threads(int(threads))

    def max_threads(self) -> int:
        return int(self.lib.cb_max_threads())

    def planes_of(self, packed: np.ndarray, n: int) -> np.ndarray:
        packed = np.ascontiguousarray(packed)
        groups = (n + 127) // 128
        planes = np.zeros((packed.shape[0], groups * 32), dtype=np.uint8)
        self.lib.cb_planes_of(_ptr(packed), packed.shape[0], n, packed.shape[1], _ptr(planes))
        return planes

    def workspace(self, n: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        groups = (n + 127) // 128
        return (np.zeros(groups * 128, dtype=np.int8), np.zeros(groups, dtype=np.int32),
                np.zeros(max(n, 1), dtype=np.float32))

    def gemv(self, x, planes, scales_f32, bias, out, accumulate: bool = False, ws=None) -> np.ndarray:
        n = x.shape[0]
        q, gsum, _ = ws if ws is not None else self.workspace(n)
        self.lib.cb_gemv(_ptr(x), n, _ptr(planes), _ptr(scales_f32), _ptr(bias), planes.shape[0], _ptr(q),
                         _ptr(gsum), _ptr(out), int(accumulate))
        return out

    def normed_gemv(self, x, weight, eps, clip, planes, scales_f32, bias, out, ws=None) -> np.ndarray:
        n = x.shape[0]
        q, gsum, work = ws if ws is not None else self.workspace(n)
        self.lib.cb_normed_gemv(_ptr(x), _ptr(weight), eps, clip, n, _ptr(work), _ptr(planes), _ptr(scales_f32),
                                _ptr(bias), planes.shape[0], _ptr(q), _ptr(gsum), _ptr(out))
        return out

    def normed_gemv_silu(self, x, weight, eps, clip, planes, scales_f32, bias, out, ws=None) -> np.ndarray:
        n = x.shape[0]
        q, gsum, work = ws if ws is not None else self.workspace(n)
        self.lib.cb_normed_gemv_silu(_ptr(x), _ptr(weight), eps, clip, n, _ptr(work), _ptr(planes),
                                     _ptr(scales_f32), _ptr(bias), out.shape[0], _ptr(q), _ptr(gsum), _ptr(out))
        return out


_ORACLE: Oracle | None = None


def oracle() -> Oracle:
    global _ORACLE
    if _ORACLE is None:
        _ORACLE = Oracle()
    return _ORACLE
