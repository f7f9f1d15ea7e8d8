"""HipBackend — Python mirror of Yule's ComputeBackend trait over libyule_hip.so.

Method names, argument order and meaning follow `yule-gpu/src/lib.rs:21-132`
(the trait) so that tests read like Yule's own backend tests
(`yule-gpu/src/cpu.rs:597-1157`).  Failures raise `YuleGpuError`, the
counterpart of `YuleError::Gpu(String)` (yule-core/src/error.rs:44).

There is no fallback: if libyule_hip.so is missing or no gfx950 device is
present, construction raises.  Buffers are `BufferHandle` (a u64 wrapper,
lib.rs:135).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .formats import DType

LIB_PATH = Path(__file__).resolve().parent / "libyule_hip.so"

# every symbol declared in include/yule_hip.h (checked by tests/test_abi.py)
_SIGS: dict[str, tuple] = {
    "yule_hip_last_error": (C.c_char_p, []),
    "yule_hip_is_available": (C.c_int, []),
    "yule_hip_create": (C.c_int, [C.c_int, C.POINTER(C.c_void_p)]),
    "yule_hip_destroy": (C.c_int, [C.c_void_p]),
    "yule_hip_name": (C.c_char_p, [C.c_void_p]),
    "yule_hip_device_info": (C.c_int, [C.c_void_p, C.c_void_p]),
    "yule_hip_allocate": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_uint64)]),
    "yule_hip_free": (C.c_int, [C.c_void_p, C.c_uint64]),
    "yule_hip_copy_to_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_uint64]),
    "yule_hip_copy_from_device": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_size_t]),
    "yule_hip_copy_buffer": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_size_t]),
    "yule_hip_copy_buffer_offset": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_size_t, C.c_size_t, C.c_size_t]),
    "yule_hip_synchronize": (C.c_int, [C.c_void_p]),
    "yule_hip_matmul": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32]),
    "yule_hip_softmax": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint32]),
    "yule_hip_rms_norm": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32, C.c_float]),
    "yule_hip_rope": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32, C.c_float, C.c_uint32, C.c_uint32]),
    "yule_hip_silu": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint32]),
    "yule_hip_element_mul": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32]),
    "yule_hip_add": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32]),
    "yule_hip_attn_score": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64] + [C.c_uint32] * 5),
    "yule_hip_attn_value": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64] + [C.c_uint32] * 5),
    "yule_hip_quantized_matmul": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32]),
    "yule_hip_quantized_matmul_multi": (C.c_int, [C.c_void_p, C.c_uint32, C.POINTER(C.c_uint64),
                                                  C.POINTER(C.c_uint64), C.POINTER(C.c_uint32), C.c_uint64,
                                                  C.c_uint32, C.c_uint32]),
    "yule_hip_dequantize": (C.c_int, [C.c_void_p, C.c_uint64, C.c_size_t, C.c_uint64, C.c_uint32, C.c_uint32]),
    "yule_hip_silu_mul": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32]),
    "yule_hip_gqa_decode_attn": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64] + [C.c_uint32] * 4),
    "yule_hip_argmax": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint64]),
    "yule_hip_quantized_gemm": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64] + [C.c_uint32] * 4),
    "yule_hip_quantized_gemm_f32": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64] + [C.c_uint32] * 4),
    "yule_hip_quantized_gemm_noalloc": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64] + [C.c_uint32] * 4),
    "yule_hip_runner_create": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p)]),
    "yule_hip_runner_destroy": (C.c_int, [C.c_void_p]),
    "yule_hip_runner_reset": (C.c_int, [C.c_void_p]),
    "yule_hip_runner_pos": (C.c_uint32, [C.c_void_p]),
    "yule_hip_runner_decode_step": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p]),
    "yule_hip_runner_prefill": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p]),
    "yule_hip_runner_prefill_batched": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p]),
    "yule_hip_runner_last_prefill_ms": (C.c_float, [C.c_void_p]),
    "yule_hip_runner_generate_greedy": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p,
                                                  C.POINTER(C.c_float)]),
    "yule_hip_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "yule_hip_gguf_close": (C.c_int, [C.c_void_p]),
    "yule_hip_gguf_header": (C.c_int, [C.c_void_p, C.POINTER(C.c_uint32)] + [C.POINTER(C.c_uint64)] * 4),
    "yule_hip_gguf_tensor": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p]),
    "yule_hip_gguf_find": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p]),
    "yule_hip_gguf_get_u32": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint32)]),
    "yule_hip_gguf_get_f64": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_double)]),
    "yule_hip_gguf_get_str": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_char_p)]),
    "yule_hip_gguf_get_array_len": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint64)]),
    "yule_hip_runner_create_from_gguf": (C.c_int, [C.c_void_p, C.c_char_p, C.c_uint32, C.POINTER(C.c_void_p)]),
    "yule_hip_read_probe": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32]),
    "yule_hip_mfma_probe": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32,
                                      C.c_uint32]),
    "yule_hip_read_probe_variant": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32,
                                              C.c_uint32, C.c_uint32]),
    "yule_hip_timer_start": (C.c_int, [C.c_void_p]),
    "yule_hip_time_empty_launches": (C.c_int, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_int, C.POINTER(C.c_float)]),
    "yule_hip_timer_stop": (C.c_int, [C.c_void_p, C.POINTER(C.c_float)]),
    "yule_hip_capture_begin": (C.c_int, [C.c_void_p]),
    "yule_hip_capture_end": (C.c_int, [C.c_void_p]),
    "yule_hip_capture_replay": (C.c_int, [C.c_void_p]),
    "yule_hip_time_qmv_ops": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_int,
                                        C.POINTER(C.c_float)]),
}


class YuleGpuError(RuntimeError):
    """YuleError::Gpu(String): a failed backend call (code + message)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class QmvOp(C.Structure):
    """yule_qmv_op: one quantized_matmul(_multi) call for time_qmv_ops."""
    _fields_ = [("n_mats", C.c_uint32), ("weights", C.c_uint64 * 4), ("outputs", C.c_uint64 * 4),
                ("n_rows", C.c_uint32 * 4), ("input", C.c_uint64), ("n_cols", C.c_uint32), ("dtype", C.c_uint32)]

    @classmethod
    def make(cls, weights, outputs, n_rows, inp, n_cols, dtype):
        n = len(weights)
        pad = lambda v, f: list(v) + [f] * (4 - n)  # noqa: E731
        return cls(n, (C.c_uint64 * 4)(*pad([_h(w) for w in weights], 0)),
                   (C.c_uint64 * 4)(*pad([_h(y) for y in outputs], 0)), (C.c_uint32 * 4)(*pad(n_rows, 0)),
                   _h(inp), n_cols, int(dtype))


class _DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("backend", C.c_uint32), ("memory_bytes", C.c_uint64),
                ("compute_units", C.c_uint32)]


@dataclass(frozen=True)
class BufferHandle:
    """BufferHandle(pub u64), yule-gpu/src/lib.rs:135."""
    id: int


@dataclass
class DeviceInfo:
    """DeviceInfo, yule-gpu/src/lib.rs:137-143."""
    name: str
    backend: str
    memory_bytes: int
    compute_units: int


_lib: C.CDLL | None = None


def load_library(path: Path | str = LIB_PATH) -> C.CDLL:
    """Load libyule_hip.so and declare every exported signature; raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path)
    if not p.exists():
        raise FileNotFoundError(f"{p} is not built: run `python -m yule_amd.build` (no CPU fallback exists)")
    lib = C.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def is_available() -> bool:
    return bool(load_library().yule_hip_is_available())


def _h(x: BufferHandle | int) -> int:
    return x.id if isinstance(x, BufferHandle) else int(x)


class HipBackend:
    """impl ComputeBackend for HipBackend — one object per device."""

    def __init__(self, device: int = 0):
        self._lib = load_library()
        be = C.c_void_p()
        self._check(self._lib.yule_hip_create(device, C.byref(be)))
        self._be = be

    # -- plumbing ------------------------------------------------------------
    def _check(self, rc: int) -> None:
        if rc != 0:
            raise YuleGpuError(rc, self._lib.yule_hip_last_error().decode(errors="replace"))

    def close(self) -> None:
        if getattr(self, "_be", None):
            self._lib.yule_hip_destroy(self._be)
            self._be = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def raw(self) -> C.c_void_p:
        return self._be

    # -- trait methods -------------------------------------------------------
    def name(self) -> str:
        return self._lib.yule_hip_name(self._be).decode()

    def device_info(self) -> DeviceInfo:
        info = _DeviceInfo()
        self._check(self._lib.yule_hip_device_info(self._be, C.byref(info)))
        return DeviceInfo(info.name.decode(errors="replace"), "hip", info.memory_bytes, info.compute_units)

    def allocate(self, size_bytes: int) -> BufferHandle:
        h = C.c_uint64()
        self._check(self._lib.yule_hip_allocate(self._be, size_bytes, C.byref(h)))
        return BufferHandle(h.value)

    def free(self, handle: BufferHandle) -> None:
        self._check(self._lib.yule_hip_free(self._be, _h(handle)))

    def copy_to_device(self, data, handle: BufferHandle) -> None:
        a = np.ascontiguousarray(data)
        self._check(self._lib.yule_hip_copy_to_device(self._be, a.ctypes.data, a.nbytes, _h(handle)))

    def copy_from_device(self, handle: BufferHandle, out: np.ndarray) -> np.ndarray:
        if not out.flags["C_CONTIGUOUS"]:
            raise ValueError("copy_from_device needs a C-contiguous array")
        self._check(self._lib.yule_hip_copy_from_device(self._be, _h(handle), out.ctypes.data, out.nbytes))
        return out

    def copy_buffer(self, src: BufferHandle, dst: BufferHandle, size: int) -> None:
        self._check(self._lib.yule_hip_copy_buffer(self._be, _h(src), _h(dst), size))

    def copy_buffer_offset(self, src, dst, src_offset: int, dst_offset: int, size: int) -> None:
        self._check(self._lib.yule_hip_copy_buffer_offset(self._be, _h(src), _h(dst), src_offset, dst_offset, size))

    def synchronize(self) -> None:
        self._check(self._lib.yule_hip_synchronize(self._be))

    def matmul(self, a, b, out, m: int, n: int, k: int) -> None:
        self._check(self._lib.yule_hip_matmul(self._be, _h(a), _h(b), _h(out), m, n, k))

    def softmax(self, inp, out, size: int) -> None:
        self._check(self._lib.yule_hip_softmax(self._be, _h(inp), _h(out), size))

    def rms_norm(self, inp, weight, out, size: int, eps: float) -> None:
        self._check(self._lib.yule_hip_rms_norm(self._be, _h(inp), _h(weight), _h(out), size, eps))

    def rope(self, q, k, pos: int, head_dim: int, freq_base: float, n_heads_q: int, n_heads_k: int) -> None:
        self._check(self._lib.yule_hip_rope(self._be, _h(q), _h(k), pos, head_dim, freq_base, n_heads_q, n_heads_k))

    def silu(self, inp, out, size: int) -> None:
        self._check(self._lib.yule_hip_silu(self._be, _h(inp), _h(out), size))

    def element_mul(self, a, b, out, size: int) -> None:
        self._check(self._lib.yule_hip_element_mul(self._be, _h(a), _h(b), _h(out), size))

    def add(self, a, b, out, size: int) -> None:
        self._check(self._lib.yule_hip_add(self._be, _h(a), _h(b), _h(out), size))

    def attn_score(self, q, k_cache, scores, head_dim, seq_len, head_offset, kv_offset, kv_stride) -> None:
        self._check(self._lib.yule_hip_attn_score(self._be, _h(q), _h(k_cache), _h(scores), head_dim, seq_len,
                                                  head_offset, kv_offset, kv_stride))

    def attn_value(self, weights, v_cache, out, head_dim, seq_len, kv_offset, kv_stride, out_offset) -> None:
        self._check(self._lib.yule_hip_attn_value(self._be, _h(weights), _h(v_cache), _h(out), head_dim, seq_len,
                                                  kv_offset, kv_stride, out_offset))

    def quantized_matmul(self, weights, inp, out, n_rows: int, n_cols: int, dtype: DType | int) -> None:
        self._check(self._lib.yule_hip_quantized_matmul(self._be, _h(weights), _h(inp), _h(out), n_rows, n_cols,
                                                        int(dtype)))

    # -- extensions ----------------------------------------------------------
    def quantized_matmul_multi(self, weights, inp, outputs, n_rows, n_cols: int, dtype: DType | int) -> None:
        n = len(weights)
        self._check(self._lib.yule_hip_quantized_matmul_multi(
            self._be, n, (C.c_uint64 * n)(*map(_h, weights)), (C.c_uint64 * n)(*map(_h, outputs)),
            (C.c_uint32 * n)(*n_rows), _h(inp), n_cols, int(dtype)))

    def dequantize(self, src, src_offset: int, dst, n_blocks: int, dtype: DType | int) -> None:
        self._check(self._lib.yule_hip_dequantize(self._be, _h(src), src_offset, _h(dst), n_blocks, int(dtype)))

    def silu_mul(self, gate, up, out, size: int) -> None:
        self._check(self._lib.yule_hip_silu_mul(self._be, _h(gate), _h(up), _h(out), size))

    def gqa_decode_attn(self, q, k_cache, v_cache, out, n_heads, n_kv_heads, head_dim, seq_len) -> None:
        self._check(self._lib.yule_hip_gqa_decode_attn(self._be, _h(q), _h(k_cache), _h(v_cache), _h(out), n_heads,
                                                       n_kv_heads, head_dim, seq_len))

    def read_probe(self, src, n_bytes: int, partials, n_partials: int) -> None:
        """One streaming-read launch over n_bytes of src (roofline probe);
        partials[i] = XOR of the words workgroup i read."""
        self._check(self._lib.yule_hip_read_probe(self._be, _h(src), n_bytes, _h(partials), n_partials))

    def mfma_probe(self, inp, out, shape: int, chains: int, n_wg: int, iters: int) -> None:
        """MFMA issue-rate probe (shape 0: 16x16x32 f16, 1: 32x32x16 f16)."""
        self._check(self._lib.yule_hip_mfma_probe(self._be, _h(inp), _h(out), shape, chains, n_wg, iters))

    def read_probe_variant(self, src, n_bytes: int, partials, n_partials: int, pattern: int, loads: int) -> None:
        """A read-probe variant (pattern 0 grid-stride, 1 per-lane runs, 2 per-workgroup
        chunks; `loads` 16-byte words in flight per lane); same partials as read_probe."""
        self._check(self._lib.yule_hip_read_probe_variant(self._be, _h(src), n_bytes, _h(partials), n_partials,
                                                          pattern, loads))

    def argmax(self, inp, n: int, out) -> None:
        self._check(self._lib.yule_hip_argmax(self._be, _h(inp), n, _h(out)))

    def quantized_gemm(self, weights, x_bf16, y, m: int, n_rows: int, n_cols: int, dtype: DType | int) -> None:
        self._check(self._lib.yule_hip_quantized_gemm(self._be, _h(weights), _h(x_bf16), _h(y), m, n_rows, n_cols,
                                                      int(dtype)))

    def quantized_gemm_f32(self, weights, x_f32, y, m: int, n_rows: int, n_cols: int, dtype: DType | int) -> None:
        """Y = X W^T for f32 X [m][n_cols] (split f16 hi + lo on the matrix cores)."""
        self._check(self._lib.yule_hip_quantized_gemm_f32(self._be, _h(weights), _h(x_f32), _h(y), m, n_rows, n_cols,
                                                          int(dtype)))

    def quantized_gemm_noalloc(self, weights, x_bf16, y, m: int, n_rows: int, n_cols: int,
                               dtype: DType | int) -> None:
        """quantized_gemm with its workspace in the library's static per-GPU array (no allocation)."""
        self._check(self._lib.yule_hip_quantized_gemm_noalloc(self._be, _h(weights), _h(x_bf16), _h(y), m, n_rows,
                                                              n_cols, int(dtype)))

    def time_qmv_ops(self, ops, iters: int, use_graph: bool = True) -> float:
        """Milliseconds (HIP events on the backend stream) for `iters` passes over
        `ops`: tuples (weights, input, output, n_rows, n_cols, dtype) for one
        matrix, or ([weights...], input, [outputs...], [n_rows...], n_cols, dtype)
        for a multi-matrix launch."""
        def mk(op):
            w, x, y, r, c, d = op
            if isinstance(w, (list, tuple)):
                return QmvOp.make(w, y, r, x, c, d)
            return QmvOp.make([w], [y], [r], x, c, d)
        arr = (QmvOp * len(ops))(*[mk(op) for op in ops])
        ms = C.c_float()
        self._check(self._lib.yule_hip_time_qmv_ops(self._be, arr, len(ops), iters, int(use_graph), C.byref(ms)))
        return ms.value

    def time_empty_launches(self, n_kernels: int, iters: int, use_graph: bool = True) -> float:
        """Milliseconds for `iters` runs of n_kernels empty-kernel launches (one
        graph replay each when use_graph), HIP events on the backend stream."""
        ms = C.c_float()
        self._check(self._lib.yule_hip_time_empty_launches(self._be, n_kernels, iters, int(use_graph),
                                                          C.byref(ms)))
        return ms.value

    def timer_start(self) -> None:
        self._check(self._lib.yule_hip_timer_start(self._be))

    def timer_stop(self) -> float:
        """Milliseconds between timer_start and now, from events on the backend stream."""
        ms = C.c_float()
        self._check(self._lib.yule_hip_timer_stop(self._be, C.byref(ms)))
        return ms.value

    def capture_begin(self) -> None:
        """Start capturing this thread's calls on the backend stream into a HIP graph."""
        self._check(self._lib.yule_hip_capture_begin(self._be))

    def capture_end(self) -> None:
        """End the capture and instantiate the graph."""
        self._check(self._lib.yule_hip_capture_end(self._be))

    def capture_replay(self) -> None:
        """Launch the captured graph on the backend stream."""
        self._check(self._lib.yule_hip_capture_replay(self._be))

    # -- conveniences ----------------------------------------------------------
    def upload(self, data) -> BufferHandle:
        a = np.ascontiguousarray(data)
        h = self.allocate(a.nbytes)
        self.copy_to_device(a, h)
        return h

    def download(self, handle, shape, dtype=np.float32) -> np.ndarray:
        return self.copy_from_device(handle, np.empty(shape, dtype=dtype))


class _LayerDesc(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("attn_norm_dtype", C.c_uint32),
                ("wq", C.c_void_p), ("wk", C.c_void_p), ("wv", C.c_void_p), ("wo", C.c_void_p),
                ("wq_dtype", C.c_uint32), ("wk_dtype", C.c_uint32), ("wv_dtype", C.c_uint32), ("wo_dtype", C.c_uint32),
                ("ffn_norm", C.c_void_p), ("ffn_norm_dtype", C.c_uint32),
                ("w_gate", C.c_void_p), ("w_up", C.c_void_p), ("w_down", C.c_void_p),
                ("w_gate_dtype", C.c_uint32), ("w_up_dtype", C.c_uint32), ("w_down_dtype", C.c_uint32)]


class _ModelDesc(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("dim", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("ff_dim", C.c_uint32), ("vocab", C.c_uint32), ("max_seq", C.c_uint32), ("norm_eps", C.c_float),
                ("rope_base", C.c_float), ("token_embd", C.c_void_p), ("token_embd_dtype", C.c_uint32),
                ("output_norm", C.c_void_p), ("output_norm_dtype", C.c_uint32), ("output", C.c_void_p),
                ("output_dtype", C.c_uint32), ("layers", C.POINTER(_LayerDesc))]


class HipRunner:
    """GpuTransformerRunner counterpart over yule_hip_runner_*: ModelRunner's
    prefill / decode_step / reset (yule-infer/src/model_runner.rs:12-17)
    plus a device-resident greedy loop."""

    def __init__(self, backend: HipBackend, model):
        self._be = backend
        self._lib = backend._lib
        cfg = model.cfg
        keep = []

        def ptr(t):
            a = np.ascontiguousarray(t.data)
            keep.append(a)
            return a.ctypes.data

        layers = (_LayerDesc * cfg.n_layers)()
        for i in range(cfg.n_layers):
            t = model.layer(i)
            L = layers[i]
            L.attn_norm, L.attn_norm_dtype = ptr(t["attn_norm"]), int(t["attn_norm"].dtype)
            L.ffn_norm, L.ffn_norm_dtype = ptr(t["ffn_norm"]), int(t["ffn_norm"].dtype)
            for fld, key in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"),
                             ("w_gate", "ffn_gate"), ("w_up", "ffn_up"), ("w_down", "ffn_down")):
                setattr(L, fld, ptr(t[key]))
                setattr(L, fld + "_dtype", int(t[key].dtype))
        e, on, o = model["token_embd.weight"], model["output_norm.weight"], model["output.weight"]
        desc = _ModelDesc(cfg.n_layers, cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.ff_dim, cfg.vocab, cfg.max_seq,
                          cfg.norm_eps, cfg.rope_base, ptr(e), int(e.dtype), ptr(on), int(on.dtype), ptr(o),
                          int(o.dtype), layers)
        r = C.c_void_p()
        backend._check(self._lib.yule_hip_runner_create(backend.raw, C.byref(desc), C.byref(r)))
        self._r = r
        self.vocab = cfg.vocab

    @classmethod
    def from_gguf(cls, backend: HipBackend, path, max_seq: int = 0) -> "HipRunner":
        """Runner over a GGUF file (yule_hip_runner_create_from_gguf); max_seq
        0 takes the file's context_length."""
        from .gguf import GgufFile
        with GgufFile(path) as g:
            vocab = g.get_u32("tokenizer.ggml.vocab_size") or g.get_array_len("tokenizer.ggml.tokens") or 0
        self = cls.__new__(cls)
        self._be, self._lib = backend, backend._lib
        r = C.c_void_p()
        backend._check(self._lib.yule_hip_runner_create_from_gguf(backend.raw, str(path).encode(), max_seq,
                                                                  C.byref(r)))
        self._r, self.vocab = r, vocab
        return self

    def close(self):
        if getattr(self, "_r", None):
            self._lib.yule_hip_runner_destroy(self._r)
            self._r = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self) -> None:
        self._be._check(self._lib.yule_hip_runner_reset(self._r))

    @property
    def pos(self) -> int:
        return int(self._lib.yule_hip_runner_pos(self._r))

    def decode_step(self, token: int) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        self._be._check(self._lib.yule_hip_runner_decode_step(self._r, token, out.ctypes.data))
        return out

    def prefill(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(self.vocab, np.float32)
        self._be._check(self._lib.yule_hip_runner_prefill(self._r, t.ctypes.data, t.size, out.ctypes.data))
        return out

    def prefill_batched(self, tokens) -> np.ndarray:
        """The tokens as one batched pass (GEMM projections); logits of the last one."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(self.vocab, np.float32)
        self._be._check(self._lib.yule_hip_runner_prefill_batched(self._r, t.ctypes.data, t.size, out.ctypes.data))
        return out

    @property
    def last_prefill_ms(self) -> float:
        """Milliseconds of the prompt pass of the last generate_greedy."""
        return float(self._lib.yule_hip_runner_last_prefill_ms(self._r))

    def generate_greedy(self, prompt, n_decode: int):
        """-> (tokens[n_decode + 1], ms per decode step)"""
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(n_decode + 1, np.uint32)
        ms = C.c_float()
        self._be._check(self._lib.yule_hip_runner_generate_greedy(self._r, p.ctypes.data, p.size, n_decode,
                                                                  out.ctypes.data, C.byref(ms)))
        return out, ms.value
