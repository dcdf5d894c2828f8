"""llmrs_hip - Python host mirror of llm.rs's operator interface on MI355X.

Binds the C ABI of ``include/llmrs_hip.h`` (``lib/libllmrs_hip.so`` plus the
gfx950 code objects it loads with ``hipModuleLoad``).  ``HipBackend`` mirrors
``trait Backend`` (reference ``src/backend.rs:15-40``) method for method;
``HipModel`` is the HBM-resident decode loop (``src/core/model.rs:17-49``
driven like ``src/main.rs:128-327`` with greedy argmax).

There is no fallback: if the shared library is missing, importing works but
the first call raises ``LlmrsError`` naming the missing file.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

LIB_DIR = Path(__file__).resolve().parent.parent / "lib"
LIB_PATH = LIB_DIR / "libllmrs_hip.so"

E_INVALID, E_DTYPE, E_HIP, E_NOINIT, E_MODULE, E_RANGE, E_OOM = -1, -2, -3, -4, -5, -6, -7


class LlmrsError(RuntimeError):
    """A non-zero return code of the C ABI (the reference panics instead)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class Device(enum.IntEnum):
    """src/backend.rs:7-12 plus the Hip variant."""
    Cpu = 0
    OpenCl = 1
    Qnn = 2
    Hip = 3


class DType(enum.IntEnum):
    """Storage kinds: src/core/tensor.rs:13-44 plus extensions."""
    F32 = 0
    F16 = 1
    Q4 = 2      # Storage::CpuQ4 (f32 scales)
    Q4_0 = 3    # fp16 scales
    Q8_0 = 4


_lib = None

_SIGS = {
    "llmrs_init": (C.c_int, [C.c_int, C.c_char_p]),
    "llmrs_shutdown": (C.c_int, []),
    "llmrs_last_error": (C.c_char_p, []),
    "llmrs_device": (C.c_int, []),
    "llmrs_name": (C.c_char_p, []),
    "llmrs_sync": (C.c_int, []),
    "llmrs_num_cus": (C.c_int, []),
    "llmrs_tensor_upload_f32": (C.c_int, [C.c_void_p, C.POINTER(C.c_size_t), C.c_int, C.POINTER(C.c_void_p)]),
    "llmrs_tensor_upload_q4": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.POINTER(C.c_void_p)]),
    "llmrs_tensor_upload_q8_0": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.POINTER(C.c_void_p)]),
    "llmrs_tensor_zeros": (C.c_int, [C.POINTER(C.c_size_t), C.c_int, C.POINTER(C.c_void_p)]),
    "llmrs_tensor_download": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "llmrs_tensor_ndim": (C.c_int, [C.c_void_p]),
    "llmrs_tensor_dims": (C.c_int, [C.c_void_p, C.POINTER(C.c_size_t)]),
    "llmrs_tensor_dtype": (C.c_int, [C.c_void_p]),
    "llmrs_tensor_free": (C.c_int, [C.c_void_p]),
    "llmrs_matmul": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p)]),
    "llmrs_matmul_transposed": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p)]),
    "llmrs_matmul_transposed_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "llmrs_matmul_slice": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.POINTER(C.c_void_p)]),
    "llmrs_add_assign": (C.c_int, [C.c_void_p, C.c_void_p]),
    "llmrs_silu_mul": (C.c_int, [C.c_void_p, C.c_void_p]),
    "llmrs_rope_inplace": (C.c_int, [C.c_void_p, C.c_size_t]),
    "llmrs_rms_norm": (C.c_int, [C.c_void_p, C.c_void_p, C.c_float, C.POINTER(C.c_void_p)]),
    "llmrs_softmax": (C.c_int, [C.c_void_p, C.POINTER(C.c_void_p)]),
    "llmrs_scale": (C.c_int, [C.c_void_p, C.c_float, C.POINTER(C.c_void_p)]),
    "llmrs_check_mul_f16": (C.c_int, [C.c_void_p, C.POINTER(C.c_void_p)]),
    "llmrs_copy_from": (C.c_int, [C.c_void_p, C.POINTER(C.c_void_p)]),
    "llmrs_model_create": (C.c_int, [C.c_void_p, C.POINTER(C.c_void_p)]),
    "llmrs_model_free": (C.c_int, [C.c_void_p]),
    "llmrs_model_get_config": (C.c_int, [C.c_void_p, C.c_void_p]),
    "llmrs_model_load_safetensors": (C.c_int, [C.c_char_p, C.c_void_p, C.POINTER(C.c_void_p)]),
    "llmrs_model_load_gguf": (C.c_int, [C.c_char_p, C.c_void_p, C.POINTER(C.c_void_p)]),
    "llmrs_model_set_embedding": (C.c_int, [C.c_void_p, C.c_void_p]),
    "llmrs_model_set_norm": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "llmrs_model_set_linear_q4": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "llmrs_model_set_linear_q8_0": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "llmrs_model_kv_write": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p]),
    "llmrs_model_kv_read": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p]),
    "llmrs_model_forward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p]),
    "llmrs_model_generate": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]),
    "llmrs_model_begin": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "llmrs_model_begin_at": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t]),
    "llmrs_model_decode_steps": (C.c_int, [C.c_void_p, C.c_size_t]),
    "llmrs_model_tokens": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "llmrs_model_set_sampling": (C.c_int, [C.c_void_p, C.c_void_p]),
    "llmrs_model_set_exact": (C.c_int, [C.c_void_p, C.c_int]),
    "llmrs_probe_expf": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p]),
    "llmrs_batch_create": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(C.c_void_p)]),
    "llmrs_batch_free": (C.c_int, [C.c_void_p]),
    "llmrs_batch_begin": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_size_t]),
    "llmrs_batch_decode_steps": (C.c_int, [C.c_void_p, C.c_size_t]),
    "llmrs_batch_tokens": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_size_t]),
    "llmrs_batch_logits": (C.c_int, [C.c_void_p, C.c_void_p]),
    "llmrs_batch_profile_step": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_void_p, C.c_int]),
    "llmrs_model_produced": (C.c_int, [C.c_void_p, C.POINTER(C.c_size_t), C.POINTER(C.c_int32)]),
    "llmrs_sample_logits": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_size_t, C.c_void_p, C.c_uint64,
                                      C.c_void_p, C.c_void_p]),
    "llmrs_model_profile_step": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_void_p, C.c_int]),
    "llmrs_model_time_linear": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "llmrs_model_profile_prefill": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_char_p,
                                               C.c_void_p, C.c_void_p, C.c_int]),
    "llmrs_model_weight_bytes": (C.c_double, [C.c_void_p]),
    "llmrs_model_decode_plan": (C.c_int, [C.c_void_p, C.c_void_p]),
    "llmrs_model_profile_stamps": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int]),
    "llmrs_model_probe_decode_layer": (C.c_int, [C.c_void_p, C.c_int, C.c_size_t, C.c_void_p, C.c_void_p]),
    "llmrs_model_probe_head": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                          C.c_void_p]),
    "llmrs_model_probe_prefill_layer": (C.c_int, [C.c_void_p, C.c_int, C.c_size_t, C.c_size_t, C.c_void_p,
                                                   C.c_void_p]),
    "llmrs_synth_q4": (C.c_int, [C.c_uint64, C.c_uint64, C.c_size_t, C.c_size_t, C.c_float, C.c_float, C.c_void_p, C.c_void_p, C.c_int]),
    "llmrs_synth_q8": (C.c_int, [C.c_uint64, C.c_uint64, C.c_size_t, C.c_size_t, C.c_float, C.c_float, C.c_void_p, C.c_void_p, C.c_int]),
    "llmrs_synth_normal": (C.c_int, [C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, C.c_float, C.c_void_p, C.c_int]),
    "llmrs_synth_tokens": (C.c_int, [C.c_uint64, C.c_uint64, C.c_size_t, C.c_int32, C.c_void_p]),
}

EXPORTED = tuple(_SIGS)


def lib() -> C.CDLL:
    """The loaded C library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise LlmrsError(E_MODULE, f"{LIB_PATH} is missing; run llm.rs_amd/build.py")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _check(rc: int) -> int:
    if rc < 0:
        raise LlmrsError(rc, lib().llmrs_last_error().decode(errors="replace"))
    return rc


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


_initialised = False


def init(device: int = 0) -> None:
    """llmrs_init: select the GPU and load the gfx950 code objects."""
    global _initialised
    if not _initialised:
        hsaco = os.environ.get("LLMRS_HSACO_DIR", str(LIB_DIR))  # alternate code objects
        _check(lib().llmrs_init(device, hsaco.encode()))
        _initialised = True


def sync() -> None:
    _check(lib().llmrs_sync())


def probe_expf(x) -> np.ndarray:
    """The device exponential of the SiLU and softmax kernels on x
    (llmrs_probe_expf): glibc's expf, bit for bit."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    _check(lib().llmrs_probe_expf(_ptr(x), x.size, _ptr(out)))
    return out


def num_cus() -> int:
    return lib().llmrs_num_cus()


class Tensor:
    """A device tensor handle (Tensor with Storage on Device::Hip)."""

    __slots__ = ("_h", "__weakref__")

    def __init__(self, handle: int):
        self._h = C.c_void_p(handle)

    @property
    def handle(self):
        return self._h

    @property
    def shape(self) -> tuple[int, ...]:
        nd = _check(lib().llmrs_tensor_ndim(self._h))
        dims = (C.c_size_t * nd)()
        _check(lib().llmrs_tensor_dims(self._h, dims))
        return tuple(int(d) for d in dims)

    @property
    def dtype(self) -> DType:
        return DType(_check(lib().llmrs_tensor_dtype(self._h)))

    def data(self) -> np.ndarray:
        """Tensor::data(): download an f32 tensor."""
        out = np.empty(self.shape, dtype=np.float32)
        _check(lib().llmrs_tensor_download(self._h, _ptr(out), out.size))
        return out

    def free(self) -> None:
        if self._h and self._h.value:
            _check(lib().llmrs_tensor_free(self._h))
            self._h = C.c_void_p(None)

    def __del__(self):
        try:
            if _lib is not None and self._h and self._h.value:
                _lib.llmrs_tensor_free(self._h)
        except Exception:
            pass

    # -- construction (Tensor::new + to_device) --------------------------
    @staticmethod
    def from_numpy(arr) -> "Tensor":
        a = np.ascontiguousarray(arr, dtype=np.float32)
        dims = (C.c_size_t * max(a.ndim, 1))(*(a.shape or (1,)))
        out = C.c_void_p()
        _check(lib().llmrs_tensor_upload_f32(_ptr(a), dims, max(a.ndim, 1), C.byref(out)))
        return Tensor(out.value)

    @staticmethod
    def from_q4(qs: np.ndarray, scales: np.ndarray, n: int, k: int) -> "Tensor":
        """Storage::CpuQ4 -> device: qs [n][k/2] reference nibble order, f32 scales."""
        qs = np.ascontiguousarray(qs, dtype=np.uint8)
        sc = np.ascontiguousarray(scales, dtype=np.float32)
        if qs.size != n * k // 2 or sc.size != n * k // 32:
            raise LlmrsError(E_INVALID, "q4 buffer sizes do not match n, k")
        out = C.c_void_p()
        _check(lib().llmrs_tensor_upload_q4(_ptr(qs), _ptr(sc), n, k, C.byref(out)))
        return Tensor(out.value)

    @staticmethod
    def from_q8_0(qs: np.ndarray, scales: np.ndarray, n: int, k: int) -> "Tensor":
        qs = np.ascontiguousarray(qs, dtype=np.int8)
        sc = np.ascontiguousarray(scales, dtype=np.float32)
        if qs.size != n * k or sc.size != n * k // 32:
            raise LlmrsError(E_INVALID, "q8 buffer sizes do not match n, k")
        out = C.c_void_p()
        _check(lib().llmrs_tensor_upload_q8_0(_ptr(qs), _ptr(sc), n, k, C.byref(out)))
        return Tensor(out.value)

    @staticmethod
    def zeros(shape) -> "Tensor":
        dims = (C.c_size_t * len(shape))(*shape)
        out = C.c_void_p()
        _check(lib().llmrs_tensor_zeros(dims, len(shape), C.byref(out)))
        return Tensor(out.value)


def _out_tensor(fn, *args) -> Tensor:
    out = C.c_void_p()
    _check(fn(*args, C.byref(out)))
    return Tensor(out.value)


class HipBackend:
    """trait Backend (src/backend.rs:15-40) on the gfx950 kernels."""

    def __init__(self, device: int = 0):
        init(device)

    def device(self) -> Device:                                   # backend.rs:17
        return Device(lib().llmrs_device())

    def name(self) -> str:                                        # backend.rs:18
        return lib().llmrs_name().decode()

    def matmul(self, a: Tensor, b: Tensor) -> Tensor:             # backend.rs:21
        return _out_tensor(lib().llmrs_matmul, a.handle, b.handle)

    def matmul_transposed(self, a: Tensor, b: Tensor) -> Tensor:  # backend.rs:24
        return _out_tensor(lib().llmrs_matmul_transposed, a.handle, b.handle)

    def matmul_transposed_noalloc(self, a: Tensor, b: Tensor, out: Tensor) -> None:
        """matmul_transposed into a pre-allocated [m, n] f32 tensor, with no
        device allocation (fixed per-device scratch; no reference
        counterpart)."""
        _check(lib().llmrs_matmul_transposed_noalloc(a.handle, b.handle, out.handle))

    def matmul_slice(self, a: Tensor, other_data, rows: int, cols: int) -> Tensor:  # backend.rs:28
        od = np.ascontiguousarray(other_data, dtype=np.float32)
        if od.size < rows * cols:
            raise LlmrsError(E_INVALID, "other_data shorter than rows*cols")
        return _out_tensor(lib().llmrs_matmul_slice, a.handle, _ptr(od), rows, cols)

    def add_assign(self, a: Tensor, b: Tensor) -> None:           # backend.rs:31
        _check(lib().llmrs_add_assign(a.handle, b.handle))

    def silu_mul(self, gate: Tensor, up: Tensor) -> None:         # backend.rs:32
        _check(lib().llmrs_silu_mul(gate.handle, up.handle))

    def rope_inplace(self, x: Tensor, start_pos: int) -> None:    # backend.rs:33
        _check(lib().llmrs_rope_inplace(x.handle, start_pos))

    def rms_norm(self, x: Tensor, weight: Tensor, eps: float) -> Tensor:  # backend.rs:36
        return _out_tensor(lib().llmrs_rms_norm, x.handle, weight.handle, C.c_float(eps))

    def softmax(self, x: Tensor) -> Tensor:                       # backend.rs:37
        return _out_tensor(lib().llmrs_softmax, x.handle)

    def scale(self, x: Tensor, value: float) -> Tensor:           # backend.rs:38
        return _out_tensor(lib().llmrs_scale, x.handle, C.c_float(value))

    def copy_from(self, t: Tensor) -> Tensor:                     # backend.rs:39
        return _out_tensor(lib().llmrs_copy_from, t.handle)

    def check_mul_f16(self, values: Tensor) -> Tensor:
        """Self-check (llmrs_check_mul_f16): mismatch counts per f16 pattern
        of the one-instruction f16 product against convert-and-multiply."""
        return _out_tensor(lib().llmrs_check_mul_f16, values.handle)


class ModelConfig(C.Structure):
    """llmrs_model_config: LlamaConfig (src/core/config.rs:3-17) plus storage."""
    _fields_ = [
        ("n_layers", C.c_int32), ("hidden", C.c_int32), ("n_heads", C.c_int32),
        ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("ffn", C.c_int32),
        ("vocab", C.c_int32), ("max_seq", C.c_int32), ("rms_eps", C.c_float),
        ("rope_theta", C.c_float), ("weight_dtype", C.c_int32), ("kv_dtype", C.c_int32),
    ]


class LoadOptions(C.Structure):
    """llmrs_load_options: KV capacity (<= 0: 2048), KV storage, weight
    storage (0: the file's own)."""
    _fields_ = [("max_seq", C.c_int32), ("kv_dtype", C.c_int32), ("weight_dtype", C.c_int32)]


MAX_EOS = 8
LLAMA3_EOS = (128001, 128009)  # main.rs:121


class Sampling(C.Structure):
    """llmrs_sampling: the token loop's sampling parameters (main.rs:42-58
    defaults: penalty 1.2 over the last 64 ids, temperature 0.8, top_p 0.9)
    and the seed that makes its draws repeat."""
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("repeat_penalty", C.c_float),
                ("penalty_window", C.c_int32), ("seed", C.c_uint64), ("n_eos", C.c_int32),
                ("eos", C.c_int32 * MAX_EOS)]

    @classmethod
    def make(cls, temperature=0.8, top_p=0.9, repeat_penalty=1.2, penalty_window=64, seed=0,
             eos=LLAMA3_EOS) -> "Sampling":
        eos = tuple(eos)
        if len(eos) > MAX_EOS:
            raise ValueError(f"at most {MAX_EOS} end-of-sequence ids")
        s = cls(float(temperature), float(top_p), float(repeat_penalty), int(penalty_window), int(seed), len(eos))
        for i, e in enumerate(eos):
            s.eos[i] = int(e)
        return s


def sample_logits(logits, history, sampling: Sampling, position: int) -> tuple[int, float]:
    """The device sampler alone on one step's logits: (drawn id, U)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    h = np.ascontiguousarray(history, dtype=np.int32)
    tok = np.zeros(1, np.int32)
    u = np.zeros(1, np.float32)
    _check(lib().llmrs_sample_logits(_ptr(lg), lg.size, _ptr(h) if h.size else None, h.size,
                                     C.byref(sampling), int(position), _ptr(tok), _ptr(u)))
    return int(tok[0]), float(u[0])


W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN, W_LM_HEAD = range(8)
N_INPUT, N_POST, N_FINAL = range(3)


@dataclass
class KernelTiming:
    name: str
    ms: float
    bytes: float


class LayerProbe(C.Structure):
    """llmrs_layer_probe: host buffers for one layer's intermediates."""
    _fields_ = [(n, C.c_void_p) for n in
                ("qkv", "xq", "xd", "ctx", "ctx_q", "ctx_d", "h", "hq", "hd", "m", "m_q", "m_d", "out")]


def _probe_arrays(cfg, rows: int) -> dict:
    H, F = cfg.hidden, cfg.ffn
    qd = cfg.n_heads * cfg.head_dim
    qr = (cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim
    f, i8 = np.float32, np.int8
    shapes = {"qkv": (qr, f), "xq": (H, i8), "xd": (H // 32, f), "ctx": (qd, f), "ctx_q": (qd, i8),
              "ctx_d": (qd // 32, f), "h": (H, f), "hq": (H, i8), "hd": (H // 32, f), "m": (F, f),
              "m_q": (F, i8), "m_d": (F // 32, f), "out": (H, f)}
    return {k: np.zeros((rows, n), t) for k, (n, t) in shapes.items()}


class HipModel:
    """The resident decode model (llmrs_model_*)."""

    def __init__(self, cfg: ModelConfig, device: int = 0):
        init(device)
        self.cfg = cfg
        h = C.c_void_p()
        _check(lib().llmrs_model_create(C.byref(cfg), C.byref(h)))
        self._h = h

    @classmethod
    def _adopt(cls, h: C.c_void_p) -> "HipModel":
        self = cls.__new__(cls)
        self._h = h
        self.cfg = ModelConfig()
        _check(lib().llmrs_model_get_config(h, C.byref(self.cfg)))
        return self

    @classmethod
    def load_safetensors(cls, path, max_seq: int = 0, kv: DType = DType.F16, device: int = 0) -> "HipModel":
        """A Hugging Face checkpoint (directory with config.json and
        model.safetensors or its shards): llmrs_model_load_safetensors."""
        init(device)
        opt = LoadOptions(int(max_seq), int(kv), 0)
        h = C.c_void_p()
        _check(lib().llmrs_model_load_safetensors(str(path).encode(), C.byref(opt), C.byref(h)))
        return cls._adopt(h)

    @classmethod
    def load_gguf(cls, path, max_seq: int = 0, kv: DType = DType.F16, weight: int = 0,
                  device: int = 0) -> "HipModel":
        """A llama-architecture GGUF file: llmrs_model_load_gguf."""
        init(device)
        opt = LoadOptions(int(max_seq), int(kv), int(weight))
        h = C.c_void_p()
        _check(lib().llmrs_model_load_gguf(str(path).encode(), C.byref(opt), C.byref(h)))
        return cls._adopt(h)

    def close(self) -> None:
        if self._h and self._h.value:
            _check(lib().llmrs_model_free(self._h))
            self._h = C.c_void_p(None)

    def __del__(self):
        try:
            if _lib is not None and self._h and self._h.value:
                _lib.llmrs_model_free(self._h)
        except Exception:
            pass

    def set_embedding(self, table: np.ndarray) -> None:
        t = np.ascontiguousarray(table, dtype=np.float32)
        _check(lib().llmrs_model_set_embedding(self._h, _ptr(t)))

    def set_norm(self, layer: int, slot: int, w: np.ndarray) -> None:
        w = np.ascontiguousarray(w, dtype=np.float32)
        _check(lib().llmrs_model_set_norm(self._h, layer, slot, _ptr(w)))

    def set_linear_q4(self, layer: int, slot: int, qs: np.ndarray, scales: np.ndarray) -> None:
        qs = np.ascontiguousarray(qs, dtype=np.uint8)
        sc = np.ascontiguousarray(scales, dtype=np.float32)
        _check(lib().llmrs_model_set_linear_q4(self._h, layer, slot, _ptr(qs), _ptr(sc)))

    def set_linear_q8_0(self, layer: int, slot: int, qs: np.ndarray, scales: np.ndarray) -> None:
        qs = np.ascontiguousarray(qs, dtype=np.int8)
        sc = np.ascontiguousarray(scales, dtype=np.float32)
        _check(lib().llmrs_model_set_linear_q8_0(self._h, layer, slot, _ptr(qs), _ptr(sc)))

    def kv_write(self, layer: int, kv_head: int, pos0: int, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        n = k.size // self.cfg.head_dim
        _check(lib().llmrs_model_kv_write(self._h, layer, kv_head, pos0, n, _ptr(k), _ptr(v)))

    def kv_read(self, layer: int, kv_head: int, pos0: int, n: int):
        k = np.empty((n, self.cfg.head_dim), np.float32)
        v = np.empty((n, self.cfg.head_dim), np.float32)
        _check(lib().llmrs_model_kv_read(self._h, layer, kv_head, pos0, n, _ptr(k), _ptr(v)))
        return k, v

    def forward(self, tokens, start_pos: int, logits: bool = True, trace: bool = False):
        """Eager forward of tokens at [start_pos, start_pos+n): (logits, next, trace)."""
        ids = np.ascontiguousarray(tokens, dtype=np.int32)
        n = ids.size
        lg = np.empty(self.cfg.vocab, np.float32) if logits else None
        nxt = np.zeros(1, np.int32)
        tr = np.empty((n, self.cfg.n_layers + 1, self.cfg.hidden), np.float32) if trace else None
        _check(lib().llmrs_model_forward(self._h, _ptr(ids), n, start_pos, _ptr(lg), _ptr(nxt), _ptr(tr)))
        return lg, int(nxt[0]), tr

    def generate(self, prompt, n_steps: int) -> np.ndarray:
        """The tokens produced; with sampling, those before a drawn
        end-of-sequence id (fewer than n_steps)."""
        ids = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_steps, np.int32)
        _check(lib().llmrs_model_generate(self._h, _ptr(ids), ids.size, n_steps, _ptr(out)))
        end = np.nonzero(out < 0)[0]
        return out[: int(end[0])] if end.size else out

    def set_sampling(self, sampling: Sampling | None) -> None:
        """Sampling (main.rs:192-305) in place of the greedy argmax; None
        restores greedy decoding."""
        _check(lib().llmrs_model_set_sampling(self._h, C.byref(sampling) if sampling is not None else None))

    def set_exact(self, on: bool = True) -> None:
        """Reference-order decode kernels (llmrs_model_set_exact): every f32
        sum in the reference CPU path's order, so logits and greedy tokens
        equal the reference's bit for bit."""
        _check(lib().llmrs_model_set_exact(self._h, 1 if on else 0))

    def produced(self) -> tuple[int, bool]:
        """(tokens produced since begin, whether an end-of-sequence id stopped the run)."""
        n = C.c_size_t(0)
        st = C.c_int32(0)
        _check(lib().llmrs_model_produced(self._h, C.byref(n), C.byref(st)))
        return int(n.value), bool(st.value)

    def begin(self, prompt, start_pos: int = 0) -> None:
        """Process the prompt at [start_pos, start_pos + n) (the cache below
        start_pos already filled) and keep the greedy state resident."""
        ids = np.ascontiguousarray(prompt, dtype=np.int32)
        _check(lib().llmrs_model_begin_at(self._h, _ptr(ids), ids.size, start_pos))

    def decode_steps(self, n: int) -> None:
        _check(lib().llmrs_model_decode_steps(self._h, n))

    def tokens(self, count: int) -> np.ndarray:
        out = np.empty(count, np.int32)
        _check(lib().llmrs_model_tokens(self._h, _ptr(out), count))
        return out

    def profile_step(self, cap: int = 4096) -> list[KernelTiming]:
        names = C.create_string_buffer(32 * cap)
        ms = np.zeros(cap, np.float32)
        by = np.zeros(cap, np.float64)
        n = _check(lib().llmrs_model_profile_step(self._h, names, _ptr(ms), _ptr(by), cap))
        raw = names.raw
        return [KernelTiming(raw[32 * i:32 * i + 32].split(b"\0")[0].decode(), float(ms[i]), float(by[i]))
                for i in range(n)]

    def time_linear(self, slot: int, reps: int = 4) -> tuple[float, float]:
        """(us per launch, algorithmic bytes per launch) of one decode GEMV
        slot over every layer, back to back."""
        us = np.zeros(1, np.float64)
        by = np.zeros(1, np.float64)
        _check(lib().llmrs_model_time_linear(self._h, slot, reps, _ptr(us), _ptr(by)))
        return float(us[0]), float(by[0])

    def profile_prefill(self, tokens, start_pos: int = 0, cap: int = 4096) -> list[KernelTiming]:
        """Per-launch timing of one batched prefill chunk; `bytes` holds FLOPs
        for the GEMM and attention launches."""
        ids = np.ascontiguousarray(tokens, dtype=np.int32)
        names = C.create_string_buffer(32 * cap)
        ms = np.zeros(cap, np.float32)
        wk = np.zeros(cap, np.float64)
        n = _check(lib().llmrs_model_profile_prefill(self._h, _ptr(ids), ids.size, start_pos, names,
                                                     _ptr(ms), _ptr(wk), cap))
        raw = names.raw
        return [KernelTiming(raw[32 * i:32 * i + 32].split(b"\0")[0].decode(), float(ms[i]), float(wk[i]))
                for i in range(n)]

    def probe_decode_layer(self, layer: int, pos: int, x: np.ndarray) -> dict:
        """One decode step of `layer` at `pos` on the row x (test probe):
        every intermediate of its kernels, as 1-D arrays (LayerProbe)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = _probe_arrays(self.cfg, 1)
        pr = LayerProbe(**{k: v.ctypes.data for k, v in out.items()})
        _check(lib().llmrs_model_probe_decode_layer(self._h, layer, pos, _ptr(x), C.byref(pr)))
        return {k: v[0] for k, v in out.items()}

    def probe_head(self, x: np.ndarray):
        """Final RMSNorm + lm_head + argmax of the row x (test probe):
        (Q8_0 codes, scales, logits, next id)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        H = self.cfg.hidden
        xq, xd = np.zeros(H, np.int8), np.zeros(H // 32, np.float32)
        lg = np.zeros(self.cfg.vocab, np.float32)
        nxt = np.zeros(1, np.int32)
        _check(lib().llmrs_model_probe_head(self._h, _ptr(x), _ptr(xq), _ptr(xd), _ptr(lg), _ptr(nxt)))
        return xq, xd, lg, int(nxt[0])

    def probe_prefill_layer(self, layer: int, start_pos: int, x: np.ndarray) -> dict:
        """The batched prefill kernels of `layer` on rows x [n][hidden] at
        positions start_pos.. (test probe): every intermediate, [n][...]."""
        x = np.ascontiguousarray(x, np.float32)
        n = x.shape[0]
        out = _probe_arrays(self.cfg, n)
        pr = LayerProbe(**{k: v.ctypes.data for k, v in out.items()})
        _check(lib().llmrs_model_probe_prefill_layer(self._h, layer, start_pos, n, _ptr(x), C.byref(pr)))
        return out

    def profile_stamps(self, layer: int, slot: int, cap: int = 1 << 16) -> np.ndarray:
        """Per-workgroup stamps of one decode GEMV in an eager step: rows of
        (start, operand ready, loop done, end, input arrived, norm factor,
        quantised [us], XCC id, HW_ID)."""
        out = np.zeros(cap, np.float64)
        n = _check(lib().llmrs_model_profile_stamps(self._h, layer, slot, _ptr(out), cap))
        return out[:n].reshape(-1, 9)

    def weight_bytes(self) -> float:
        return float(lib().llmrs_model_weight_bytes(self._h))

    def decode_plan(self) -> dict:
        """How a decode step runs its attention (llmrs_model_decode_plan)."""
        out = np.zeros(4, np.int32)
        _check(lib().llmrs_model_decode_plan(self._h, _ptr(out)))
        return {"nsplit": int(out[0]), "tile_waves": int(out[1]), "xcd_local": bool(out[2]),
                "exact": bool(out[3])}


# -- seeded synthetic inputs (llmrs_synth_*) ------------------------------
class HipBatch:
    """B sequences of one model decoding together (llmrs_batch_*)."""

    def __init__(self, model: HipModel, batch: int):
        self.model = model
        self.batch = batch
        h = C.c_void_p()
        _check(lib().llmrs_batch_create(model._h, int(batch), C.byref(h)))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().llmrs_batch_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def begin(self, slot: int, prompt) -> None:
        ids = np.ascontiguousarray(prompt, dtype=np.int32)
        _check(lib().llmrs_batch_begin(self._h, int(slot), _ptr(ids), ids.size))

    def decode_steps(self, n: int) -> None:
        _check(lib().llmrs_batch_decode_steps(self._h, int(n)))

    def tokens(self, slot: int, count: int) -> np.ndarray:
        out = np.empty(count, np.int32)
        _check(lib().llmrs_batch_tokens(self._h, int(slot), _ptr(out), count))
        return out

    def logits(self) -> np.ndarray:
        out = np.empty((self.batch, self.model.cfg.vocab), np.float32)
        _check(lib().llmrs_batch_logits(self._h, _ptr(out)))
        return out

    def profile_step(self, cap: int = 8192) -> list[KernelTiming]:
        names = C.create_string_buffer(32 * cap)
        ms = np.zeros(cap, np.float32)
        work = np.zeros(cap, np.float64)
        n = _check(lib().llmrs_batch_profile_step(self._h, names, _ptr(ms), _ptr(work), cap))
        raw = names.raw
        return [KernelTiming(raw[32 * i:32 * i + 32].split(b"\0")[0].decode(), float(ms[i]), float(work[i]))
                for i in range(n)]


def synth_q4(seed: int, tid: int, n: int, k: int, lo: float, hi: float, threads: int = 0):
    qs = np.empty(n * k // 2, np.uint8)
    sc = np.empty(n * k // 32, np.float32)
    _check(lib().llmrs_synth_q4(seed, tid, n, k, lo, hi, _ptr(qs), _ptr(sc), threads))
    return qs, sc


def synth_q8(seed: int, tid: int, n: int, k: int, lo: float, hi: float, threads: int = 0):
    qs = np.empty(n * k, np.int8)
    sc = np.empty(n * k // 32, np.float32)
    _check(lib().llmrs_synth_q8(seed, tid, n, k, lo, hi, _ptr(qs), _ptr(sc), threads))
    return qs, sc


def synth_normal(seed: int, tid: int, count: int, mean: float, std: float, threads: int = 0):
    out = np.empty(count, np.float32)
    _check(lib().llmrs_synth_normal(seed, tid, count, mean, std, _ptr(out), threads))
    return out


def synth_tokens(seed: int, tid: int, count: int, vocab: int) -> np.ndarray:
    out = np.empty(count, np.int32)
    _check(lib().llmrs_synth_tokens(seed, tid, count, vocab, _ptr(out)))
    return out
