"""CPU oracle: ctypes view of oracle/build/liboracle.so (the C restatement of
Yule's CPU path, see the per-function citations in oracle/*.c).

TEST INFRASTRUCTURE ONLY.  Importable by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, and only as the checker / the timed CPU
baseline; the product (libyule_hip.so and yule_amd's compute path) never
imports, links or calls it.

Parity pins: tests/test_oracle.py checks every function here against the
reference's own known-answer tests, the reference's hand-written Q4_K AVX2
assembly (oracle/_ref/, built from the reference sources when present),
exhaustive bit-pattern sweeps and closed-form special cases.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "build" / "liboracle.so"
REF_Q4K_ASM = HERE / "_ref" / "libyule_q4k_asm.so"

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 2, 8, 12, 13, 14, 15
GEOM = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_K: (256, 292)}

_lib = None
_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)


class Layer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("wq", C.c_void_p), ("wk", C.c_void_p), ("wv", C.c_void_p),
                ("wo", C.c_void_p), ("wq_t", C.c_int), ("wk_t", C.c_int), ("wv_t", C.c_int), ("wo_t", C.c_int),
                ("ffn_norm", C.c_void_p), ("w_gate", C.c_void_p), ("w_up", C.c_void_p), ("w_down", C.c_void_p),
                ("w_gate_t", C.c_int), ("w_up_t", C.c_int), ("w_down_t", C.c_int)]


class Model(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("dim", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("ff_dim", C.c_uint32), ("vocab", C.c_uint32), ("max_seq", C.c_uint32), ("norm_eps", C.c_float),
                ("rope_base", C.c_float), ("token_embd", C.c_void_p), ("token_embd_t", C.c_int),
                ("output_norm", C.c_void_p), ("output", C.c_void_p), ("output_t", C.c_int),
                ("layers", C.POINTER(Layer))]


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise FileNotFoundError(f"{LIB} missing: run `make -C oracle`")
        L = C.CDLL(str(LIB))
        L.yo_f16_to_f32.argtypes = [C.c_uint16]
        L.yo_f16_to_f32.restype = C.c_float
        L.yo_extract_q4k_scales_mins.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
        for n in ("yo_dequant_q4_0", "yo_dequant_q8_0", "yo_dequant_q4_k", "yo_dequant_q6_k", "yo_dequant_q5_k",
                  "yo_dequant_q8_k"):
            getattr(L, n).argtypes = [C.c_void_p, C.c_void_p]
        for n in ("yo_vec_dot_q4_0", "yo_vec_dot_q8_0", "yo_vec_dot_q4_k", "yo_vec_dot_q6_k", "yo_vec_dot_q5_k"):
            getattr(L, n).argtypes = [C.c_void_p, C.c_void_p]
            getattr(L, n).restype = C.c_float
        L.yo_dequant_rows.argtypes = [C.c_int, C.c_void_p, C.c_size_t, C.c_void_p]
        L.yo_vec_dot_block.argtypes = [C.c_int, C.c_void_p, C.c_void_p, _f32p]
        L.yo_vec_dot_block_scalar.argtypes = [C.c_int, C.c_void_p, C.c_void_p, _f32p]
        L.yo_qmv_scalar.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32]
        L.yo_qmv_f64.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32]
        L.yo_qmv.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_int]
        L.yo_have_avx2.restype = C.c_int
        L.yo_set_q4k_dot.argtypes = [C.c_void_p]
        L.yo_argmax.argtypes = [C.c_void_p, C.c_uint32]
        L.yo_argmax.restype = C.c_uint32
        L.yo_rope_table.argtypes = [C.c_uint32, C.c_uint32, C.c_float, C.c_void_p, C.c_void_p]
        L.yo_runner_new.argtypes = [C.POINTER(Model), C.c_int]
        L.yo_runner_new.restype = C.c_void_p
        L.yo_runner_free.argtypes = [C.c_void_p]
        L.yo_runner_reset.argtypes = [C.c_void_p]
        L.yo_runner_forward.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p]
        L.yo_runner_pos.argtypes = [C.c_void_p]
        L.yo_runner_pos.restype = C.c_uint32
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def f16_to_f32(bits: int) -> float:
    return lib().yo_f16_to_f32(bits)


def extract_q4k_scales_mins(q12: bytes | np.ndarray):
    q = np.frombuffer(bytes(q12), dtype=np.uint8).copy()
    sc = np.zeros(8, np.uint8)
    mn = np.zeros(8, np.uint8)
    lib().yo_extract_q4k_scales_mins(_ptr(q), _ptr(sc), _ptr(mn))
    return sc, mn


def dequant(dtype: int, data: np.ndarray) -> np.ndarray:
    """dequant_block over every block of `data` (u8) -> f32."""
    bs, bb = GEOM[dtype]
    data = np.ascontiguousarray(data, dtype=np.uint8)
    nb = data.size // bb
    out = np.empty(nb * bs, np.float32)
    if lib().yo_dequant_rows(dtype, _ptr(data), nb, _ptr(out)):
        raise ValueError("unsupported dtype")
    return out


def vec_dot(dtype: int, block: np.ndarray, act: np.ndarray, scalar: bool = True) -> float:
    r = C.c_float()
    fn = lib().yo_vec_dot_block_scalar if scalar else lib().yo_vec_dot_block
    block = np.ascontiguousarray(block, dtype=np.uint8)
    act = np.ascontiguousarray(act, dtype=np.float32)
    if fn(dtype, _ptr(block), _ptr(act), C.byref(r)):
        raise ValueError("unsupported dtype")
    return r.value


def qmv_scalar(dtype, w, x, n_rows, n_cols) -> np.ndarray:
    """CpuBackend::quantized_matmul (yule-gpu/src/cpu.rs:544-590)."""
    y = np.empty(n_rows, np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().yo_qmv_scalar(dtype, _ptr(w), _ptr(x), _ptr(y), n_rows, n_cols)
    return y


def qmv_f64(dtype, w, x, n_rows, n_cols) -> np.ndarray:
    """f64-accumulated dot of the bit-exact dequantized weights."""
    y = np.empty(n_rows, np.float64)
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().yo_qmv_f64(dtype, _ptr(w), _ptr(x), _ptr(y), n_rows, n_cols)
    return y


def qmv(dtype, w, x, n_rows, n_cols, n_threads: int = 0) -> np.ndarray:
    """model_runner.rs:152-244 qmv: AVX2 vec_dot, per-call thread row split."""
    y = np.empty(n_rows, np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().yo_qmv(dtype, _ptr(w), _ptr(x), _ptr(y), n_rows, n_cols, n_threads)
    return y


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(lib().yo_argmax(_ptr(v), v.size))


def rope_table(max_seq: int, rot_dim: int, base: float):
    half = rot_dim // 2
    c = np.empty(max_seq * half, np.float32)
    s = np.empty(max_seq * half, np.float32)
    lib().yo_rope_table(max_seq, rot_dim, base, _ptr(c), _ptr(s))
    return c, s


def q4k_asm():
    """The reference's hand-written AVX2 Q4_K dot (yule-core/src/kernels/
    q4k_gemv_avx2.S) built by `make -C oracle ref`, or None if not built."""
    if not REF_Q4K_ASM.exists():
        return None
    L = C.CDLL(str(REF_Q4K_ASM))
    L.yule_q4k_gemv_avx2.argtypes = [C.c_void_p, C.c_void_p]
    L.yule_q4k_gemv_avx2.restype = C.c_float
    return L.yule_q4k_gemv_avx2


def set_q4k_dot(fn) -> None:
    """Run the AVX2 path's Q4_K block dot through `fn` (q4k_asm(): the
    reference's assembly kernel, as its own AVX2 build does), or through the
    Rust-fallback restatement again with None."""
    lib().yo_set_q4k_dot(C.cast(fn, C.c_void_p) if fn is not None else None)


class Runner:
    """TransformerRunner restatement (oracle/runner.c) over a model dict from
    yule_amd.model (tensors by GGUF name)."""

    # formats the reference's CPU vec_dot dispatch handles (simd/scalar.rs:4-22);
    # a model with any other matrix format cannot run on Yule's CPU path
    VEC_DOT = (2, 8, 12, 13, 14)   # Q4_0, Q8_0, Q4_K, Q5_K, Q6_K

    def __init__(self, model, n_threads: int = 0):
        cfg = model.cfg
        for name, t in model.tensors.items():
            if t.data.ndim and name != "token_embd.weight" and t.dtype not in (0, 1) and int(t.dtype) not in self.VEC_DOT:
                raise ValueError(f"{name}: dtype {int(t.dtype)} has no vec_dot in the reference (scalar.rs:4-22)")
        self._keep = []
        layers = (Layer * cfg.n_layers)()
        for i in range(cfg.n_layers):
            t = model.layer(i)
            L = layers[i]
            for fld, key in (("attn_norm", "attn_norm"), ("ffn_norm", "ffn_norm")):
                setattr(L, fld, self._hold(t[key].data))
            for fld, key in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"),
                             ("w_gate", "ffn_gate"), ("w_up", "ffn_up"), ("w_down", "ffn_down")):
                setattr(L, fld, self._hold(t[key].data))
                setattr(L, fld + "_t", int(t[key].dtype))
        m = Model(cfg.n_layers, cfg.dim, cfg.n_heads, cfg.n_kv_heads, cfg.ff_dim, cfg.vocab, cfg.max_seq,
                  cfg.norm_eps, cfg.rope_base, self._hold(model["token_embd.weight"].data),
                  int(model["token_embd.weight"].dtype), self._hold(model["output_norm.weight"].data),
                  self._hold(model["output.weight"].data), int(model["output.weight"].dtype), layers)
        self._layers = layers
        self._model = m
        self.vocab = cfg.vocab
        self._r = lib().yo_runner_new(C.byref(m), n_threads)
        if not self._r:
            raise MemoryError("yo_runner_new failed")

    def _hold(self, a: np.ndarray) -> int:
        a = np.ascontiguousarray(a)
        self._keep.append(a)
        return a.ctypes.data

    def forward(self, token: int) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        if lib().yo_runner_forward(self._r, token, _ptr(out)):
            raise RuntimeError("oracle forward failed (context length exceeded or bad token)")
        return out

    def reset(self) -> None:
        lib().yo_runner_reset(self._r)

    @property
    def pos(self) -> int:
        return lib().yo_runner_pos(self._r)

    def __del__(self):
        if getattr(self, "_r", None):
            lib().yo_runner_free(self._r)
            self._r = None
