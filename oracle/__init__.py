"""ctypes binding of the CPU oracle (oracle/oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py - as the tests' parity reference and the timed CPU baseline,
never as a product path.  Build with ``make -C oracle``.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_lib = None

_I64 = C.c_int64
_P = C.c_void_p
_SIGS = {
    "orc_set_threads": (None, [C.c_int]),
    "orc_get_threads": (C.c_int, []),
    "orc_set_arch": (None, [C.c_int]),
    "orc_get_arch": (C.c_int, []),
    "orc_record_codes": (None, [C.c_int]),
    "orc_set_attn_f64": (None, [C.c_int]),
    "orc_recorded_codes": (_I64, [_P, _I64]),
    "orc_inject_codes": (None, [_P, _I64, C.c_float]),
    "orc_injected_stats": (None, [_P, _P, _P, _P]),
    "orc_gemv_codes": (None, [_P, _P, _I64, _I64, _P, _P, _I64, C.c_int, _P]),
    "orc_model_attention": (C.c_int, [_P, C.c_int, _P, _I64, _I64, _P]),
    "orc_quantize_row_q8_0": (None, [_P, _I64, _P, _P]),
    "orc_quantize_q4": (None, [_P, _I64, _P, _P]),
    "orc_dequantize_q4": (None, [_P, _P, _I64, _P]),
    "orc_q4_block_isum": (C.c_int32, [_P, _P]),
    "orc_q4_block_isum_scalar": (C.c_int32, [_P, _P]),
    "orc_matmul_transposed_q4": (None, [_P, _I64, _I64, _P, _P, _I64, _P]),
    "orc_matmul_transposed_q8w": (None, [_P, _I64, _I64, _P, _P, _I64, _P]),
    "orc_matmul_transposed_f32": (None, [_P, _I64, _I64, _P, _I64, _P]),
    "orc_matmul": (None, [_P, _I64, _I64, _P, _I64, _P]),
    "orc_matmul_slice": (None, [_P, _I64, _I64, _P, _I64, _P]),
    "orc_add_assign": (None, [_P, _P, _I64]),
    "orc_silu_mul": (None, [_P, _P, _I64]),
    "orc_expf": (None, [_P, _I64, _P]),
    "orc_rope_inplace": (None, [_P, _I64, _I64, _I64]),
    "orc_rms_norm": (None, [_P, _I64, _I64, _P, C.c_float, _P]),
    "orc_softmax": (None, [_P, _I64, _I64, _P]),
    "orc_scale": (None, [_P, _I64, C.c_float, _P]),
    "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
    "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
    "orc_argmax": (_I64, [_P, _I64, _P]),
    "orc_sample": (C.c_int32, [_P, _I64, _P, _I64, C.c_float, C.c_float, C.c_float, _I64, C.c_float,
                               C.c_int32, _P]),
    "orc_model_create": (_P, [_P]),
    "orc_model_free": (None, [_P]),
    "orc_model_set_embedding": (C.c_int, [_P, _P]),
    "orc_model_set_norm": (C.c_int, [_P, C.c_int, C.c_int, _P]),
    "orc_model_set_linear_q4": (C.c_int, [_P, C.c_int, C.c_int, _P, _P]),
    "orc_model_set_linear_q8": (C.c_int, [_P, C.c_int, C.c_int, _P, _P]),
    "orc_model_kv_write": (C.c_int, [_P, C.c_int, C.c_int, _I64, _I64, _P, _P]),
    "orc_model_kv_read": (C.c_int, [_P, C.c_int, C.c_int, _I64, _I64, _P, _P]),
    "orc_model_forward": (C.c_int, [_P, _P, _I64, _I64, _P, C.c_int, _P]),
    "orc_model_generate": (C.c_int, [_P, _P, _I64, _I64, _P, _P]),
}


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        h = C.CDLL(str(LIB_PATH))
        for n, (r, a) in _SIGS.items():
            f = getattr(h, n)
            f.restype = r
            f.argtypes = a
        _lib = h
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


def set_arch(arch: int) -> None:
    """Test-only: restate the reference's x86-64 build (0, the default) or
    its aarch64 build (1: NEON summation orders of the Q4 GEMV, f32 dot and
    saxpy, cpu.rs:461-619,747-886)."""
    lib().orc_set_arch(arch)


def set_attn_f64(on: bool) -> None:
    """Test-only: the attention's scores, softmax and P.V summed in float64
    (rounded to f32 once), the rest of the arithmetic unchanged."""
    lib().orc_set_attn_f64(1 if on else 0)


def record_codes(on: bool) -> None:
    """Test-only: start (clearing) or stop recording every Q8_0 code."""
    lib().orc_record_codes(1 if on else 0)


def recorded_codes() -> np.ndarray:
    n = lib().orc_recorded_codes(None, 0)
    out = np.empty(n, np.int8)
    lib().orc_recorded_codes(_p(out), n)
    return out


def inject_codes(codes, tol: float = 0.0) -> None:
    """Test-only: replay forward passes with these Q8_0 codes (in the call
    order of quantize_row_q8_0) instead of the oracle's own rounding; None
    stops.  Differing codes are checked against `tol` (injected_stats)."""
    if codes is None:
        lib().orc_inject_codes(None, 0, 0.0)
        return
    codes = np.ascontiguousarray(codes, np.int8)
    inject_codes._held = codes
    lib().orc_inject_codes(_p(codes), codes.size, float(tol))


def injected_stats() -> dict:
    """Codes taken, codes differing from the oracle's own, differing codes
    not one step away at a rounding midpoint (within tol, or past the end of
    the given codes), and the largest midpoint distance of a differing code."""
    t, d, b = (C.c_int64(), C.c_int64(), C.c_int64())
    m = C.c_float()
    lib().orc_injected_stats(C.byref(t), C.byref(d), C.byref(b), C.byref(m))
    return {"taken": t.value, "differ": d.value, "bad": b.value, "max_dist": m.value}


def gemv_codes(xq, xd, w, scales, n, q8w=False):
    """The reference block loop over already-quantised activation rows
    (xq [m][k] int8, xd [m][k/32]) for Q4 (reference nibble order) or Q8
    weight codes: [m][n]."""
    xq = np.ascontiguousarray(xq, np.int8)
    if xq.ndim == 1:
        xq = xq[None]
    m, k = xq.shape
    xd = _f32(xd).reshape(m, k // 32)
    w = np.ascontiguousarray(w, np.int8 if q8w else np.uint8)
    out = np.empty((m, n), np.float32)
    lib().orc_gemv_codes(_p(xq), _p(xd), m, k, _p(w), _p(_f32(scales)), n, 1 if q8w else 0, _p(out))
    return out


def threads() -> int:
    return lib().orc_get_threads()


def quantize_row_q8_0(x):
    x = _f32(x).ravel()
    q = np.empty(x.size, np.int8)
    d = np.empty(x.size // 32, np.float32)
    lib().orc_quantize_row_q8_0(_p(x), x.size, _p(q), _p(d))
    return q, d


def quantize_q4(x):
    x = _f32(x).ravel()
    qs = np.empty(x.size // 2, np.uint8)
    sc = np.empty(x.size // 32, np.float32)
    lib().orc_quantize_q4(_p(x), x.size, _p(qs), _p(sc))
    return qs, sc


def dequantize_q4(qs, scales, count):
    out = np.empty(count, np.float32)
    lib().orc_dequantize_q4(_p(np.ascontiguousarray(qs, np.uint8)), _p(_f32(scales)), count, _p(out))
    return out


def q4_block_isum(q4, a, scalar=False):
    q4 = np.ascontiguousarray(q4, np.uint8)
    a = np.ascontiguousarray(a, np.int8)
    f = lib().orc_q4_block_isum_scalar if scalar else lib().orc_q4_block_isum
    return int(f(_p(q4), _p(a)))


def matmul_transposed_q4(a, qs, scales, n):
    a = _f32(a)
    m, k = a.shape
    out = np.empty((m, n), np.float32)
    lib().orc_matmul_transposed_q4(_p(a), m, k, _p(np.ascontiguousarray(qs, np.uint8)), _p(_f32(scales)), n, _p(out))
    return out


def matmul_transposed_q8w(a, qs, scales, n):
    a = _f32(a)
    m, k = a.shape
    out = np.empty((m, n), np.float32)
    lib().orc_matmul_transposed_q8w(_p(a), m, k, _p(np.ascontiguousarray(qs, np.int8)), _p(_f32(scales)), n, _p(out))
    return out


def matmul_transposed_f32(a, b):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[0]
    out = np.empty((m, n), np.float32)
    lib().orc_matmul_transposed_f32(_p(a), m, k, _p(b), n, _p(out))
    return out


def matmul(a, b):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    out = np.empty((m, n), np.float32)
    lib().orc_matmul(_p(a), m, k, _p(b), n, _p(out))
    return out


def matmul_slice(a, other, rows):
    a, other = _f32(a), _f32(other)
    m, k = a.shape
    out = np.empty((m, rows), np.float32)
    lib().orc_matmul_slice(_p(a), m, k, _p(other), rows, _p(out))
    return out


def add_assign(a, b):
    a = _f32(a).copy()
    lib().orc_add_assign(_p(a), _p(_f32(b)), a.size)
    return a


def silu_mul(g, u):
    g = _f32(g).copy()
    lib().orc_silu_mul(_p(g), _p(_f32(u)), g.size)
    return g


def expf(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_expf(_p(x), x.size, _p(out))
    return out


def rope_inplace(x, start_pos):
    x = _f32(x).copy()
    lib().orc_rope_inplace(_p(x), x.size, x.shape[-1], start_pos)
    return x


def rms_norm(x, w, eps):
    x = _f32(x)
    out = np.empty_like(x)
    dim = x.shape[-1]
    lib().orc_rms_norm(_p(x), x.size // dim, dim, _p(_f32(w)), eps, _p(out))
    return out


def softmax(x):
    x = _f32(x)
    out = np.empty_like(x)
    dim = x.shape[-1]
    lib().orc_softmax(_p(x), x.size // dim, dim, _p(out))
    return out


def scale(x, v):
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_scale(_p(x), x.size, v, _p(out))
    return out


def f32_to_f16_bits(x: float) -> int:
    return int(lib().orc_f32_to_f16(x))


def argmax(x):
    x = _f32(x)
    m = C.c_float()
    i = lib().orc_argmax(_p(x), x.size, C.byref(m))
    return int(i), float(m.value)


def sample(logits, history, penalty, temperature, top_p, window, u, candidate=-1):
    """The reference's sampling (main.rs:192-305) for the draw u: (id,
    whether `candidate` is acceptable - equal, or within the rounding of the
    reference's f32 running sums)."""
    x = _f32(logits)
    h = np.ascontiguousarray(history, np.int32)
    acc = C.c_int32(0)
    t = lib().orc_sample(_p(x), x.size, _p(h) if h.size else None, h.size, float(penalty),
                         float(temperature), float(top_p), int(window), float(u), int(candidate),
                         C.byref(acc))
    return int(t), bool(acc.value)


class OrcConfig(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int32), ("hidden", C.c_int32), ("n_heads", C.c_int32),
        ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("ffn", C.c_int32),
        ("vocab", C.c_int32), ("max_seq", C.c_int32), ("rms_eps", C.c_float),
        ("rope_theta", C.c_float), ("weight_dtype", C.c_int32), ("kv_dtype", C.c_int32),
    ]


class OracleModel:
    """The reference model on the CPU; weight arrays are borrowed (kept here)."""

    def __init__(self, n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq,
                 rms_eps=1e-5, rope_theta=500000.0, weight_dtype=3, kv_dtype=0):
        self.cfg = OrcConfig(n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq,
                             rms_eps, rope_theta, weight_dtype, kv_dtype)
        self._h = lib().orc_model_create(C.byref(self.cfg))
        if not self._h:
            raise ValueError("oracle rejected the configuration")
        self._keep = []

    @classmethod
    def from_spec(cls, spec, max_seq=None):
        return cls(spec.n_layers, spec.hidden, spec.n_heads, spec.n_kv_heads, spec.head_dim, spec.ffn,
                   spec.vocab, max_seq or spec.max_seq, spec.rms_eps, spec.rope_theta, int(spec.weight),
                   1 if int(spec.kv) == 1 else 0)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_model_free(self._h)
            self._h = None

    def _hold(self, *arrs):
        self._keep.extend(arrs)

    def set_embedding(self, t):
        t = _f32(t)
        self._hold(t)
        assert lib().orc_model_set_embedding(self._h, _p(t)) == 0

    def set_norm(self, layer, slot, w):
        w = _f32(w)
        self._hold(w)
        assert lib().orc_model_set_norm(self._h, layer, slot, _p(w)) == 0

    def set_linear_q4(self, layer, slot, qs, scales):
        qs, sc = np.ascontiguousarray(qs, np.uint8), _f32(scales)
        self._hold(qs, sc)
        assert lib().orc_model_set_linear_q4(self._h, layer, slot, _p(qs), _p(sc)) == 0

    def set_linear_q8(self, layer, slot, qs, scales):
        qs, sc = np.ascontiguousarray(qs, np.int8), _f32(scales)
        self._hold(qs, sc)
        assert lib().orc_model_set_linear_q8(self._h, layer, slot, _p(qs), _p(sc)) == 0

    def kv_write(self, layer, kv_head, pos0, k, v):
        k, v = _f32(k), _f32(v)
        n = k.size // self.cfg.head_dim
        assert lib().orc_model_kv_write(self._h, layer, kv_head, pos0, n, _p(k), _p(v)) == 0

    def kv_read(self, layer, kv_head, pos0, n):
        k = np.empty((n, self.cfg.head_dim), np.float32)
        v = np.empty((n, self.cfg.head_dim), np.float32)
        assert lib().orc_model_kv_read(self._h, layer, kv_head, pos0, n, _p(k), _p(v)) == 0
        return k, v

    def attention(self, layer, qkv, start_pos):
        """Attention of `layer` given Q|K|V projections [seq][(nq+2nkv)hd]
        (before RoPE) at positions start_pos..: appends K/V, returns ctx."""
        qkv = _f32(qkv)
        if qkv.ndim == 1:
            qkv = qkv[None]
        seq = qkv.shape[0]
        ctx = np.empty((seq, self.cfg.n_heads * self.cfg.head_dim), np.float32)
        rc = lib().orc_model_attention(self._h, layer, _p(qkv), seq, start_pos, _p(ctx))
        if rc:
            raise ValueError("oracle attention failed")
        return ctx

    def forward(self, tokens, start_pos, all_rows=False, trace=False):
        ids = np.ascontiguousarray(tokens, np.int32)
        n = ids.size
        lg = np.empty((n if all_rows else 1, self.cfg.vocab), np.float32)
        tr = np.empty((n, self.cfg.n_layers + 1, self.cfg.hidden), np.float32) if trace else None
        rc = lib().orc_model_forward(self._h, _p(ids), n, start_pos, _p(lg), int(all_rows), _p(tr))
        if rc:
            raise ValueError("oracle forward failed")
        return (lg if all_rows else lg[0]), tr

    def generate(self, prompt, n_steps):
        ids = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_steps, np.int32)
        mg = np.empty(n_steps, np.float32)
        rc = lib().orc_model_generate(self._h, _p(ids), ids.size, n_steps, _p(out), _p(mg))
        if rc:
            raise ValueError("oracle generate failed")
        return out, mg

    def load(self, w):
        """Borrow every tensor of a synthetic.Weights."""
        from llmrs_hip import DType  # noqa: WPS433 (lazy: package path set by caller)
        spec = w.spec
        if w.embed is not None:
            self.set_embedding(w.embed)
        self.set_norm(-1, 2, w.final_norm)
        put = self.set_linear_q8 if spec.weight == DType.Q8_0 else self.set_linear_q4
        put(-1, 7, *w.lm_head)
        for l in range(spec.n_layers):
            self.set_norm(l, 0, w.norms[l][0])
            self.set_norm(l, 1, w.norms[l][1])
            for s, arrs in w.linears[l].items():
                put(l, s, *arrs)
