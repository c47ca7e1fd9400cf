"""Python host API of the MI355X deterministic integer transformer path.

A thin ctypes layer over include/detgpu.h (libdetgpu.so). Names mirror the
reference's operator API for this path (src/shared/numerics/det_kernels.rs):
``det_linear_into``, ``det_linear_slab``, ``rms_norm``, ``rope_rotate_pairs``,
``attention`` and the routine-level ``Session.prefill`` / ``Session.decode``
(prefill_layer / decode_transition). There is no CPU fallback: loading fails
loudly when the HIP library is missing.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import weakref
import os
import pathlib
from typing import Optional

import numpy as np

PKG_DIR = pathlib.Path(__file__).resolve().parents[1]
LIB_PATH = PKG_DIR / "build" / "libdetgpu.so"

DET_STORAGE_INT8, DET_STORAGE_I16, DET_STORAGE_I32 = 8, 16, 32
DET_EW_ADD, DET_EW_GELU_MUL, DET_EW_SCALE, DET_EW_SOFTCAP = 0, 1, 2, 3
DET_COMMIT_NONE, DET_COMMIT_ACTIVATIONS, DET_COMMIT_KV, DET_COMMIT_ALL = 0, 1, 2, 3
DET_DECODE_PER_OP = 0x100
DET_DECODE_EAGER = 0x200


class DetError(RuntimeError):
    """A non-zero status from the C ABI (1 invalid argument, 2 contract violation, 3 runtime)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"detgpu status {status}: {message}")
        self.status = status


class TextConfig(C.Structure):
    """det_text_config_t: the raw Gemma text_config (gemma/io.rs:60-96)."""

    _fields_ = [
        ("enable_moe_block", C.c_int32),
        ("hidden_activation_is_gelu_pytorch_tanh", C.c_int32),
        ("has_final_logit_softcapping", C.c_int32),
        ("final_logit_softcapping", C.c_float),
        ("has_global_head_dim", C.c_int32),
        ("global_head_dim", C.c_uint64),
        ("head_dim", C.c_uint64),
        ("hidden_size", C.c_uint64),
        ("has_hidden_size_per_layer_input", C.c_int32),
        ("hidden_size_per_layer_input", C.c_uint64),
        ("num_layer_types", C.c_uint64),
        ("layer_types", C.POINTER(C.c_int32)),
        ("has_num_global_key_value_heads", C.c_int32),
        ("num_global_key_value_heads", C.c_uint64),
        ("num_attention_heads", C.c_uint64),
        ("num_hidden_layers", C.c_uint64),
        ("num_key_value_heads", C.c_uint64),
        ("rms_norm_eps", C.c_float),
        ("has_full_partial_rotary_factor", C.c_int32),
        ("full_partial_rotary_factor", C.c_float),
        ("has_full_rope_theta", C.c_int32),
        ("full_rope_theta", C.c_float),
        ("has_sliding_rope_theta", C.c_int32),
        ("sliding_rope_theta", C.c_float),
        ("has_rope_theta", C.c_int32),
        ("rope_theta", C.c_float),
        ("sliding_window", C.c_uint64),
        ("has_tie_word_embeddings", C.c_int32),
        ("tie_word_embeddings", C.c_int32),
        ("vocab_size", C.c_uint64),
        ("has_vocab_size_per_layer_input", C.c_int32),
        ("vocab_size_per_layer_input", C.c_uint64),
        ("has_attention_k_eq_v", C.c_int32),
        ("attention_k_eq_v", C.c_int32),
        ("has_num_kv_shared_layers", C.c_int32),
        ("num_kv_shared_layers", C.c_uint64),
        ("bidirectional_all", C.c_int32),
    ]

    @classmethod
    def from_json(cls, config_json: dict) -> "TextConfig":
        """Fills the struct from a config.json dict (serde field set of GemmaTextConfigFile)."""
        tc = config_json.get("text_config", config_json)
        c = cls()
        c.enable_moe_block = int(bool(tc["enable_moe_block"]))
        c.hidden_activation_is_gelu_pytorch_tanh = int(tc["hidden_activation"] == "gelu_pytorch_tanh")

        def opt(key, conv):
            v = tc.get(key)
            if v is not None:
                setattr(c, "has_" + key, 1)
                setattr(c, key, conv(v))

        opt("final_logit_softcapping", float)
        opt("global_head_dim", int)
        c.head_dim = int(tc["head_dim"])
        c.hidden_size = int(tc["hidden_size"])
        opt("hidden_size_per_layer_input", int)
        types = [int(t == "sliding_attention") for t in tc["layer_types"]]
        c._types = (C.c_int32 * len(types))(*types)  # keeps the storage alive with the struct
        c.num_layer_types = len(types)
        c.layer_types = C.cast(c._types, C.POINTER(C.c_int32))
        opt("num_global_key_value_heads", int)
        c.num_attention_heads = int(tc["num_attention_heads"])
        c.num_hidden_layers = int(tc["num_hidden_layers"])
        c.num_key_value_heads = int(tc["num_key_value_heads"])
        c.rms_norm_eps = float(np.float32(tc["rms_norm_eps"]))
        rp = tc.get("rope_parameters") or {}
        full, sliding = rp.get("full_attention") or {}, rp.get("sliding_attention") or {}
        if full.get("partial_rotary_factor") is not None:
            c.has_full_partial_rotary_factor, c.full_partial_rotary_factor = 1, float(full["partial_rotary_factor"])
        if full.get("rope_theta") is not None:
            c.has_full_rope_theta, c.full_rope_theta = 1, float(full["rope_theta"])
        if sliding.get("rope_theta") is not None:
            c.has_sliding_rope_theta, c.sliding_rope_theta = 1, float(sliding["rope_theta"])
        if rp.get("rope_theta") is not None:
            c.has_rope_theta, c.rope_theta = 1, float(rp["rope_theta"])
        c.sliding_window = int(tc["sliding_window"])
        opt("tie_word_embeddings", int)
        c.vocab_size = int(tc["vocab_size"])
        opt("vocab_size_per_layer_input", int)
        opt("attention_k_eq_v", int)
        opt("num_kv_shared_layers", int)
        c.bidirectional_all = int(tc.get("use_bidirectional_attention") == "all")
        return c


class PrefillResult(C.Structure):
    _fields_ = [("embedding", C.c_char * 65), ("final_hidden", C.c_char * 65), ("logits", C.c_char * 65),
                ("kv", C.c_char * 65), ("next_token", C.c_uint32)]


class DecodeResult(C.Structure):
    _fields_ = [("activation", C.c_char * 65), ("logits", C.c_char * 65), ("kv", C.c_char * 65),
                ("next_token", C.c_uint32)]


class Sampling(C.Structure):
    """det_sampling_t: SamplingConfig (shared/api/input.rs:45-50)."""

    _fields_ = [("has_max_new_tokens", C.c_int32), ("max_new_tokens", C.c_uint64),
                ("has_temperature", C.c_int32), ("temperature", C.c_float),
                ("has_top_k", C.c_int32), ("top_k", C.c_uint64),
                ("has_top_p", C.c_int32), ("top_p", C.c_float)]


DETOKENIZE_FN = C.CFUNCTYPE(C.c_int64, C.POINTER(C.c_uint32), C.c_uint64, C.c_void_p, C.c_size_t, C.c_void_p)


class TraceRequest(C.Structure):
    _fields_ = [("prompt_text", C.c_char_p), ("prompt_token_ids", C.POINTER(C.c_uint32)),
                ("prompt_token_count", C.c_uint64), ("sampling", Sampling), ("prompt_checkpoint", C.c_int32),
                ("terminal_checkpoint", C.c_char_p), ("prefill_token_range_width", C.c_uint64),
                ("decode_layer_range_width", C.c_uint64), ("detokenize", DETOKENIZE_FN),
                ("detokenize_user", C.c_void_p)]


class TraceError(DetError):
    """A failed traced run; .artifact holds the trace of the checkpoints before the failure."""

    def __init__(self, status: int, message: str, artifact: bytes):
        super().__init__(status, message)
        self.artifact = artifact


@dataclasses.dataclass(frozen=True)
class CheckpointDivergence:
    """The first divergence between a claimed trace and a replay
    (shared/api/audit.rs:85-110); None fields are the reference's None."""

    entry_index: int
    checkpoint_id: str
    occurrence: int
    claimed_checkpoint_id: Optional[str] = None
    claimed_commitment: Optional[str] = None
    replayed_commitment: Optional[str] = None


@dataclasses.dataclass(frozen=True)
class AuditOutcome:
    """challenger::audit's outcome (audit.rs:124-138): divergence None is
    NoDivergence. detour is the --raster-at spec of the divergent routine
    occurrence (None for structural divergences and routines without a raster
    detour); the raster detour run itself belongs to the raster executor."""

    divergence: Optional[CheckpointDivergence] = None
    detour: Optional[str] = None

    @property
    def diverged(self) -> bool:
        return self.divergence is not None

    @classmethod
    def from_json(cls, text: bytes) -> "AuditOutcome":
        import json

        o = json.loads(text)
        if not o["diverged"]:
            return cls()
        return cls(CheckpointDivergence(**o["divergence"]), o["detour"])


def _outcome_cap(*traces: bytes) -> int:
    # every string in the outcome comes from one of the traces or is a
    # replayed 64-hex commitment; escaping takes at most 6 bytes per byte
    return 1024 + 6 * sum(len(t) for t in traces)


def locate_divergence(claimed: bytes, replayed: bytes) -> AuditOutcome:
    """locate_first_divergence (runtime/roles/challenger.rs:136-183) between two
    serialized trace artifacts, with the detour spec of the divergence."""
    L = lib()
    cap = _outcome_cap(claimed, replayed)
    buf = C.create_string_buffer(cap)
    n, d = C.c_size_t(), C.c_int32()
    st = L.det_trace_locate_divergence(claimed, len(claimed), replayed, len(replayed), buf, cap, C.byref(n),
                                       C.byref(d))
    if st != 0:
        raise DetError(st, (L.det_ctx_last_error(None) or b"").decode())
    return AuditOutcome.from_json(buf.raw[:n.value])


_LIB = None
C = C  # ctypes, re-exported for callers that pass raw pointers


def library_path() -> pathlib.Path:
    return pathlib.Path(os.environ.get("DETGPU_LIB", str(LIB_PATH)))


def lib() -> C.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.exists():
        raise RuntimeError(f"libdetgpu.so not found at {path}; build it with `make -C raster-inference_amd` "
                           "(the det path has no CPU fallback)")
    L = C.CDLL(str(path))
    P, u64, i32p = C.c_void_p, C.c_uint64, C.POINTER(C.c_int32)
    sig = {
        "det_version": (C.c_char_p, []),
        "det_ctx_create": (C.c_int, [C.c_int, C.POINTER(P)]),
        "det_ctx_destroy": (None, [P]),
        "det_ctx_last_error": (C.c_char_p, [P]),
        "det_ctx_synchronize": (C.c_int, [P]),
        "det_device_alloc": (C.c_int, [P, C.c_size_t, C.POINTER(P)]),
        "det_device_free": (C.c_int, [P, P]),
        "det_memcpy_h2d": (C.c_int, [P, P, P, C.c_size_t]),
        "det_memcpy_d2h": (C.c_int, [P, P, P, C.c_size_t]),
        "det_memcpy_d2d": (C.c_int, [P, P, P, C.c_size_t]),
        "det_event_create": (C.c_int, [P, C.POINTER(P)]),
        "det_event_record": (C.c_int, [P, P]),
        "det_event_elapsed_ms": (C.c_int, [P, P, P, C.POINTER(C.c_float)]),
        "det_event_destroy": (None, [P]),
        "det_ctx_capture_begin": (C.c_int, [P]),
        "det_ctx_capture_end": (C.c_int, [P, C.POINTER(P)]),
        "det_graph_launch": (C.c_int, [P, P]),
        "det_graph_destroy": (None, [P]),
        "det_matrix_upload": (C.c_int, [P, u64, u64, C.c_int, P, P, C.POINTER(P)]),
        "det_matrix_info": (C.c_int, [P, C.POINTER(u64), C.POINTER(u64), C.POINTER(C.c_int)]),
        "det_matrix_free": (None, [P]),
        "det_linear": (C.c_int, [P, P, P, P]),
        "det_linear_acc_i64": (C.c_int, [P, P, P, P]),
        "det_linear_slab": (C.c_int, [P, P, u64, P, P]),
        "det_rms_norm": (C.c_int, [P, P, u64, u64, P, C.c_int64]),
        "det_rope": (C.c_int, [P, P, u64, u64, u64, u64, u64, C.c_int64, u64, u64]),
        "det_attention_causal": (C.c_int, [P, P, P, P, u64, u64, u64, u64, u64, u64, P]),
        "det_argmax_first": (C.c_int, [P, P, u64, C.POINTER(C.c_uint32)]),
        "det_argmax_first_noalloc": (C.c_int, [P, P, u64, P]),
        "det_elementwise": (C.c_int, [P, C.c_int, P, P, u64, C.c_int32]),
        "det_model_create": (C.c_int, [P, C.POINTER(TextConfig), C.POINTER(P)]),
        "det_model_set_tensor": (C.c_int, [P, C.c_char_p, u64, P, C.c_int, P, P]),
        "det_model_load_detwgt": (C.c_int, [P, P, C.c_size_t]),
        "det_model_finalize": (C.c_int, [P]),
        "det_model_fused_decode": (C.c_int, [P]),
        "det_model_free": (None, [P]),
        "det_session_create": (C.c_int, [P, u64, C.POINTER(P)]),
        "det_session_clone": (C.c_int, [P, C.POINTER(P)]),
        "det_session_free": (None, [P]),
        "det_session_prefill": (C.c_int, [P, P, u64, C.c_uint32, C.POINTER(PrefillResult)]),
        "det_session_decode": (C.c_int, [P, C.c_uint32, C.c_uint32, C.POINTER(DecodeResult)]),
        "det_session_decode_batch": (C.c_int, [P, u64, P, C.c_uint32, P]),
        "det_session_logits": (C.c_int, [P, i32p, u64]),
        "det_session_position": (C.c_int, [P, C.POINTER(u64)]),
        "det_capture": (C.c_int, [P, P, u64, u64, C.c_char_p, C.c_size_t]),
        "det_trace_run": (C.c_int, [P, C.POINTER(TraceRequest), C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t),
                                    C.POINTER(C.c_int32)]),
        "det_trace_locate_divergence": (C.c_int, [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t, C.c_char_p,
                                                  C.c_size_t, C.POINTER(C.c_size_t), C.POINTER(C.c_int32)]),
        "det_audit_trace": (C.c_int, [P, C.POINTER(TraceRequest), C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t,
                                      C.POINTER(C.c_size_t), C.POINTER(C.c_int32)]),
        "det_synthetic_int8": (C.c_int, [u64, u64, u64, C.c_int32, P, P]),
        "det_synthetic_i16": (C.c_int, [u64, u64, u64, C.c_int32, P]),
        "det_scratch_create": (C.c_int, [P, C.POINTER(P)]),
        "det_scratch_free": (None, [P]),
        "det_kv_create": (C.c_int, [P, u64, u64, C.POINTER(P)]),
        "det_kv_clone": (C.c_int, [P, C.POINTER(P)]),
        "det_kv_free": (None, [P]),
        "det_kv_info": (C.c_int, [P, C.POINTER(u64), C.POINTER(u64), C.POINTER(u64), C.POINTER(C.c_int32)]),
        "det_kv_read_logical": (C.c_int, [P, P, P, u64]),
        "det_kv_commitment": (C.c_int, [P, u64, C.c_char_p, C.POINTER(C.c_int32)]),
        "det_embed_tokens": (C.c_int, [P, P, P, u64, P]),
        "det_prefill_ple_inputs": (C.c_int, [P, P, u64, P, u64, P, P, C.POINTER(C.c_int32)]),
        "det_decode_ple_input": (C.c_int, [P, P, C.c_uint32, P, u64, P, C.POINTER(C.c_int32)]),
        "det_layer_prefill": (C.c_int, [P, P, u64, P, u64, P, P, P, P]),
        "det_layer_decode": (C.c_int, [P, P, u64, P, P, P, P, u64, P]),
        "det_hidden_to_logits": (C.c_int, [P, P, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = L
    return L


def exported_symbols() -> list[str]:
    """Names of the C ABI entry points this wrapper binds."""
    lib()
    return [n for n in dir(_LIB) if n.startswith("det_")]


def _ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data)


def synthetic_int8(seed: int, rows: int, cols: int, scale_max: int):
    """Counter-hash int8 weights + row scales (det_synthetic_int8; same values as
    synthetic.fast_int8_matrix, generated by multi-threaded native code)."""
    q = np.empty((rows, cols), dtype=np.int8)
    s = np.empty(rows, dtype=np.int32)
    st = lib().det_synthetic_int8(seed & ((1 << 64) - 1), rows, cols, scale_max, _ptr(q), _ptr(s))
    if st:
        raise DetError(st, lib().det_ctx_last_error(None).decode())
    return q, s


def synthetic_i16(seed: int, rows: int, cols: int, lim: int) -> np.ndarray:
    """Counter-hash i16 Wgt bits (det_synthetic_i16; same values as
    synthetic.fast_i16_matrix, generated by multi-threaded native code)."""
    w = np.empty((rows, cols), dtype=np.int16)
    st = lib().det_synthetic_i16(seed & ((1 << 64) - 1), rows, cols, lim, _ptr(w))
    if st:
        raise DetError(st, lib().det_ctx_last_error(None).decode())
    return w


class Context:
    """det_ctx_t: one device, one HIP stream."""

    def __init__(self, device: int = 0):
        self.lib = lib()
        h = C.c_void_p()
        st = self.lib.det_ctx_create(device, C.byref(h))
        if st:
            raise DetError(st, self.lib.det_ctx_last_error(None).decode())
        self.handle = h
        # objects holding device resources of this context, released (sessions
        # first) before the context itself so none outlives it
        self._children = weakref.WeakSet()

    def _adopt(self, obj) -> None:
        self._children.add(obj)

    def check(self, status: int) -> None:
        if status:
            raise DetError(status, self.lib.det_ctx_last_error(self.handle).decode())

    def close(self) -> None:
        if getattr(self, "handle", None):
            order = {"Graph": 0, "Session": 0, "KvCache": 0, "Scratch": 0, "Model": 1, "Matrix": 2, "DeviceBuffer": 3,
                     "Event": 4}
            for child in sorted(list(getattr(self, "_children", ())), key=lambda c: order.get(type(c).__name__, 5)):
                child._release()
            self.lib.det_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self) -> None:
        self.check(self.lib.det_ctx_synchronize(self.handle))

    # -- memory ---------------------------------------------------------------
    def alloc(self, nbytes: int) -> "DeviceBuffer":
        p = C.c_void_p()
        self.check(self.lib.det_device_alloc(self.handle, nbytes, C.byref(p)))
        return DeviceBuffer(self, p.value, nbytes)

    def to_device(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = self.alloc(max(a.nbytes, 1))
        b.dtype, b.shape = a.dtype, a.shape
        if a.nbytes:
            self.check(self.lib.det_memcpy_h2d(self.handle, C.c_void_p(b.ptr), _ptr(a), a.nbytes))
        return b

    def empty(self, shape, dtype=np.int32) -> "DeviceBuffer":
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        b = self.alloc(max(n, 1))
        b.dtype, b.shape = np.dtype(dtype), tuple(np.atleast_1d(shape))
        return b

    # -- events ---------------------------------------------------------------
    def event(self) -> "Event":
        return Event(self)

    def capture(self, calls) -> "Graph":
        """Records calls() (issued on the context stream) as a graph to replay."""
        self.check(self.lib.det_ctx_capture_begin(self.handle))
        try:
            calls()
        except BaseException:
            # a failed C call has ended the capture already; anything else
            # leaves it open: end it and drop the partial graph
            h = C.c_void_p()
            if self.lib.det_ctx_capture_end(self.handle, C.byref(h)) == 0 and h.value:
                self.lib.det_graph_destroy(h)
            raise
        h = C.c_void_p()
        self.check(self.lib.det_ctx_capture_end(self.handle, C.byref(h)))
        return Graph(self, h)

    # -- weights --------------------------------------------------------------
    def upload_matrix(self, values: np.ndarray, row_scale: np.ndarray | None = None) -> "Matrix":
        return Matrix(self, values, row_scale)

    # -- operator API (det_kernels.rs) ------------------------------------------
    def det_linear_into(self, w: "Matrix", act: "DeviceBuffer", out: "DeviceBuffer") -> None:
        self.check(self.lib.det_linear(self.handle, w.handle, C.c_void_p(act.ptr), C.c_void_p(out.ptr)))

    def det_linear_acc_i64(self, w: "Matrix", act: "DeviceBuffer", out: "DeviceBuffer") -> None:
        self.check(self.lib.det_linear_acc_i64(self.handle, w.handle, C.c_void_p(act.ptr), C.c_void_p(out.ptr)))

    def det_linear_slab(self, w: "Matrix", m: int, act: "DeviceBuffer", out: "DeviceBuffer") -> None:
        self.check(self.lib.det_linear_slab(self.handle, w.handle, m, C.c_void_p(act.ptr), C.c_void_p(out.ptr)))

    def rms_norm(self, x: "DeviceBuffer", rows: int, cols: int, weight: "DeviceBuffer | None", eps: int) -> None:
        wp = C.c_void_p(weight.ptr) if weight is not None else None
        self.check(self.lib.det_rms_norm(self.handle, C.c_void_p(x.ptr), rows, cols, wp, eps))

    def rope_rotate_pairs(self, x: "DeviceBuffer", rows: int, heads: int, head_dim: int, rotary_dim: int,
                          freq_base_dim: int, base: int, pos0: int, pos_step: int = 1) -> None:
        self.check(self.lib.det_rope(self.handle, C.c_void_p(x.ptr), rows, heads, head_dim, rotary_dim,
                                     freq_base_dim, base, pos0, pos_step))

    def attention(self, q, k, v, n_queries, n_rows, num_heads, num_kv_heads, head_dim, window, out) -> None:
        self.check(self.lib.det_attention_causal(self.handle, C.c_void_p(q.ptr), C.c_void_p(k.ptr),
                                                 C.c_void_p(v.ptr), n_queries, n_rows, num_heads, num_kv_heads,
                                                 head_dim, window, C.c_void_p(out.ptr)))

    def argmax_first(self, x: "DeviceBuffer", n: int) -> int:
        r = C.c_uint32()
        self.check(self.lib.det_argmax_first(self.handle, C.c_void_p(x.ptr), n, C.byref(r)))
        return r.value

    def argmax_first_noalloc(self, x: "DeviceBuffer", n: int, index: "DeviceBuffer") -> None:
        """Allocation-free argmax_first into the device word `index` (no synchronization)."""
        self.check(self.lib.det_argmax_first_noalloc(self.handle, C.c_void_p(x.ptr), n, C.c_void_p(index.ptr)))

    def elementwise(self, op: int, x: "DeviceBuffer", y: "DeviceBuffer | None", n: int, scalar: int = 0) -> None:
        yp = C.c_void_p(y.ptr) if y is not None else None
        self.check(self.lib.det_elementwise(self.handle, op, C.c_void_p(x.ptr), yp, n, scalar))


class DeviceBuffer:
    def __init__(self, ctx: Context, ptr: int, nbytes: int):
        self.ctx, self.ptr, self.nbytes = ctx, ptr, nbytes
        self.dtype, self.shape = np.dtype(np.uint8), (nbytes,)
        ctx._adopt(self)

    def numpy(self, dtype=None, shape=None) -> np.ndarray:
        dtype = np.dtype(dtype or self.dtype)
        shape = shape or self.shape
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            self.ctx.check(self.ctx.lib.det_memcpy_d2h(self.ctx.handle, _ptr(out), C.c_void_p(self.ptr), out.nbytes))
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        self.ctx.check(self.ctx.lib.det_memcpy_h2d(self.ctx.handle, C.c_void_p(self.ptr), _ptr(a), a.nbytes))

    def free(self) -> None:
        if self.ptr and self.ctx.handle:
            self.ctx.check(self.ctx.lib.det_device_free(self.ctx.handle, C.c_void_p(self.ptr)))
        self.ptr = 0

    def _release(self) -> None:
        if self.ptr and self.ctx.handle:
            self.ctx.lib.det_device_free(self.ctx.handle, C.c_void_p(self.ptr))
        self.ptr = 0

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


class Event:
    def __init__(self, ctx: Context):
        self.ctx = ctx
        h = C.c_void_p()
        ctx.check(ctx.lib.det_event_create(ctx.handle, C.byref(h)))
        self.handle = h
        ctx._adopt(self)

    def record(self) -> "Event":
        self.ctx.check(self.ctx.lib.det_event_record(self.ctx.handle, self.handle))
        return self

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        self.ctx.check(self.ctx.lib.det_event_elapsed_ms(self.ctx.handle, self.handle, end.handle, C.byref(ms)))
        return ms.value

    def _release(self) -> None:
        if self.handle and self.ctx.handle:
            self.ctx.lib.det_event_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


class Graph:
    def __init__(self, ctx: Context, handle):
        self.ctx = ctx
        self.handle = handle
        ctx._adopt(self)

    def launch(self) -> None:
        self.ctx.check(self.ctx.lib.det_graph_launch(self.ctx.handle, self.handle))

    def _release(self) -> None:
        if self.handle and self.ctx.handle:
            self.ctx.lib.det_graph_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


class Matrix:
    """DetNumMatrix on the device (int8 x row scale, or i16 / i32 Wgt bits)."""

    def __init__(self, ctx: Context, values: np.ndarray, row_scale: np.ndarray | None = None):
        self.ctx = ctx
        v = np.ascontiguousarray(values)
        width = {np.dtype(np.int8): 8, np.dtype(np.int16): 16, np.dtype(np.int32): 32}[v.dtype]
        rs = None
        if width == 8:
            if row_scale is None:
                raise ValueError("int8 matrices need a row scale")
            self._rs = np.ascontiguousarray(row_scale, dtype=np.int32)
            rs = _ptr(self._rs)
        h = C.c_void_p()
        ctx.check(ctx.lib.det_matrix_upload(ctx.handle, v.shape[0], v.shape[1], width, _ptr(v), rs, C.byref(h)))
        self.handle = h
        self.rows, self.cols = v.shape
        ctx._adopt(self)

    @property
    def storage(self) -> int:
        s = C.c_int()
        self.ctx.lib.det_matrix_info(self.handle, None, None, C.byref(s))
        return s.value

    def _release(self) -> None:
        if self.handle and self.ctx.handle:
            self.ctx.lib.det_matrix_free(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


class Model:
    """Gemma4TransformerModel in det mode, resident on the device."""

    def __init__(self, ctx: Context, config_json: dict):
        self.ctx = ctx
        self.cfg = TextConfig.from_json(config_json)
        h = C.c_void_p()
        ctx.check(ctx.lib.det_model_create(ctx.handle, C.byref(self.cfg), C.byref(h)))
        self.handle = h
        ctx._adopt(self)

    def load_detwgt(self, data: bytes) -> "Model":
        buf = np.frombuffer(data, dtype=np.uint8)
        self.ctx.check(self.ctx.lib.det_model_load_detwgt(self.handle, _ptr(buf), buf.size))
        return self

    def set_tensor(self, name: str, values: np.ndarray, row_scale: np.ndarray | None = None) -> None:
        v = np.ascontiguousarray(values)
        width = {np.dtype(np.int8): 8, np.dtype(np.int16): 16, np.dtype(np.int32): 32}[v.dtype]
        dims = np.asarray(v.shape, dtype=np.uint64)
        rs = None if row_scale is None else _ptr(np.ascontiguousarray(row_scale, dtype=np.int32))
        self.ctx.check(self.ctx.lib.det_model_set_tensor(self.handle, name.encode(), v.ndim, _ptr(dims), width,
                                                         _ptr(v), rs))

    def finalize(self) -> "Model":
        self.ctx.check(self.ctx.lib.det_model_finalize(self.handle))
        return self

    @property
    def fused_decode(self) -> bool:
        """Whether decode steps run the graph-captured fused step."""
        return self.ctx.lib.det_model_fused_decode(self.handle) == 1

    def session(self, max_tokens: int) -> "Session":
        return Session(self, max_tokens)

    def capture(self, prompt, decode_steps: int) -> dict:
        import json

        ids = np.asarray(prompt, dtype=np.uint32)
        buf = C.create_string_buffer((1 << 20) + decode_steps * 512)
        self.ctx.check(self.ctx.lib.det_capture(self.handle, _ptr(ids), ids.size, decode_steps, buf, len(buf)))
        return json.loads(buf.value.decode())

    def _trace_request(self, prompt_text, prompt_token_ids, max_new_tokens, temperature, top_k, top_p, detokenize,
                       prompt_checkpoint, terminal_checkpoint, prefill_token_range_width, decode_layer_range_width):
        """det_trace_request_t plus what must outlive the call (ids, callback)
        and the list that collects the detokenizer's exceptions."""
        ids = np.ascontiguousarray(prompt_token_ids, dtype=np.uint32)
        sp = Sampling(max_new_tokens is not None, max_new_tokens or 0, temperature is not None,
                      temperature if temperature is not None else 0.0, top_k is not None, top_k or 0,
                      top_p is not None, top_p if top_p is not None else 0.0)
        errors = []

        def detok(ptr_ids, n, out, cap, _user):
            try:
                text = detokenize([ptr_ids[i] for i in range(n)]).encode()
                if len(text) < cap:
                    C.memmove(out, text + b"\0", len(text) + 1)
                return len(text)
            except Exception as e:  # noqa: BLE001 - reported through the status
                errors.append(e)
                return -1

        cb = DETOKENIZE_FN(detok) if detokenize is not None else DETOKENIZE_FN()
        req = TraceRequest(prompt_text.encode(), ids.ctypes.data_as(C.POINTER(C.c_uint32)), ids.size, sp,
                           int(prompt_checkpoint), terminal_checkpoint.encode() if terminal_checkpoint else None,
                           prefill_token_range_width, decode_layer_range_width, cb, None)
        return req, (ids, cb), errors

    def _error_message(self, errors) -> str:
        msg = (self.ctx.lib.det_ctx_last_error(self.ctx.handle) or b"").decode()
        return msg + (f" ({errors[0]!r})" if errors else "")

    def trace(self, prompt_text: str, prompt_token_ids, max_new_tokens=None, temperature=1.0, top_k=None,
              top_p=None, detokenize=None, prompt_checkpoint: bool = True, terminal_checkpoint=None,
              prefill_token_range_width: int = 0, decode_layer_range_width: int = 0):
        """Runs the native deterministic sequence with checkpoint commitment and
        returns (trace artifact bytes, paused). detokenize(ids) -> str decodes
        generated ids (special tokens skipped). None means an Option left unset."""
        req, _keep, errors = self._trace_request(prompt_text, prompt_token_ids, max_new_tokens, temperature, top_k,
                                                 top_p, detokenize, prompt_checkpoint, terminal_checkpoint,
                                                 prefill_token_range_width, decode_layer_range_width)
        # each committed checkpoint is one line of about 100 bytes
        n_ids, layers, new = _keep[0].size, int(self.cfg.num_hidden_layers), max_new_tokens or 0
        pw, dw = max(prefill_token_range_width or n_ids, 1), max(decode_layer_range_width or layers, 1)
        entries = 4 + layers * (-(-n_ids // pw) + 1) + new * (2 + -(-layers // dw)) + 1
        cap = entries * 128 + 4096
        while True:
            buf = C.create_string_buffer(cap)
            n = C.c_size_t()
            paused = C.c_int32()
            st = self.ctx.lib.det_trace_run(self.handle, C.byref(req), buf, cap, C.byref(n), C.byref(paused))
            if st == 1 and n.value + 1 > cap and b"buffer too small" in (self.ctx.lib.det_ctx_last_error(self.ctx.handle) or b""):
                cap = n.value + 1
                continue
            break
        artifact = buf.raw[:n.value]
        if st != 0:
            raise TraceError(st, self._error_message(errors), artifact)
        return artifact, bool(paused.value)

    def claim(self, prompt_text: str, prompt_token_ids, max_new_tokens=None, temperature=1.0, top_k=None,
              top_p=None, detokenize=None) -> bytes:
        """claimer::run (runtime/roles/claimer.rs:34-61): the full committed
        trace artifact of the request, prompt.prepare included."""
        artifact, paused = self.trace(prompt_text, prompt_token_ids, max_new_tokens, temperature, top_k, top_p,
                                      detokenize)
        if paused:
            raise DetError(1, "claimer run paused unexpectedly")
        return artifact

    def audit(self, prompt_text: str, prompt_token_ids, claimed_trace: bytes, max_new_tokens=None,
              temperature=1.0, top_k=None, top_p=None, detokenize=None) -> AuditOutcome:
        """challenger::audit (runtime/roles/challenger.rs:55-113): replays the
        request on the GPU under the claimer policy and locates the first
        divergence of claimed_trace from the replay."""
        req, _keep, errors = self._trace_request(prompt_text, prompt_token_ids, max_new_tokens, temperature, top_k,
                                                 top_p, detokenize, True, None, 0, 0)
        cap = _outcome_cap(claimed_trace)
        buf = C.create_string_buffer(cap)
        n, d = C.c_size_t(), C.c_int32()
        st = self.ctx.lib.det_audit_trace(self.handle, C.byref(req), claimed_trace, len(claimed_trace), buf, cap,
                                          C.byref(n), C.byref(d))
        if st != 0:
            raise DetError(st, self._error_message(errors))
        return AuditOutcome.from_json(buf.raw[:n.value])

    def _release(self) -> None:
        if self.handle and self.ctx.handle:
            self.ctx.lib.det_model_free(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


class Session:
    """One sequence's KV caches + scratch (TransformerDecodeState on the device)."""

    def __init__(self, model: Model, max_tokens: int, _handle=None):
        self.model, self.ctx = model, model.ctx
        if _handle is None:
            h = C.c_void_p()
            self.ctx.check(self.ctx.lib.det_session_create(model.handle, max_tokens, C.byref(h)))
            _handle = h
        self.handle = _handle
        self.ctx._adopt(self)

    def prefill(self, token_ids, flags: int = DET_COMMIT_ALL) -> PrefillResult:
        ids = np.asarray(token_ids, dtype=np.uint32)
        r = PrefillResult()
        self.ctx.check(self.ctx.lib.det_session_prefill(self.handle, _ptr(ids), ids.size, flags, C.byref(r)))
        return r

    def decode(self, token: int, flags: int = DET_COMMIT_ALL) -> DecodeResult:
        r = DecodeResult()
        self.ctx.check(self.ctx.lib.det_session_decode(self.handle, int(token), flags, C.byref(r)))
        return r

    def position(self) -> int:
        p = C.c_uint64()
        self.ctx.check(self.ctx.lib.det_session_position(self.handle, C.byref(p)))
        return p.value

    def logits(self, vocab: int) -> np.ndarray:
        out = np.empty(vocab, dtype=np.int32)
        self.ctx.check(self.ctx.lib.det_session_logits(self.handle, out.ctypes.data_as(C.POINTER(C.c_int32)), vocab))
        return out

    def clone(self) -> "Session":
        h = C.c_void_p()
        self.ctx.check(self.ctx.lib.det_session_clone(self.handle, C.byref(h)))
        return Session(self.model, 0, _handle=h)

    def _release(self) -> None:
        if self.handle and self.ctx.handle:
            self.ctx.lib.det_session_free(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass
def _dptr(buf) -> C.c_void_p:
    return C.c_void_p(buf.ptr) if buf is not None else None


class Scratch:
    """det_scratch_t: row buffers of the layer-level operators (DetDecodeScratch)."""

    def __init__(self, model: "Model"):
        self.model, self.ctx = model, model.ctx
        h = C.c_void_p()
        self.ctx.check(self.ctx.lib.det_scratch_create(model.handle, C.byref(h)))
        self.handle = h
        self.ctx._adopt(self)

    def _release(self) -> None:
        if self.handle and self.ctx.handle:
            self.ctx.lib.det_scratch_free(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


class KvCache:
    """det_kv_t: one layer's LayerKvCache on the device."""

    def __init__(self, model: "Model", layer: int, max_tokens: int, _handle=None):
        self.model, self.ctx, self.layer = model, model.ctx, layer
        if _handle is None:
            h = C.c_void_p()
            self.ctx.check(self.ctx.lib.det_kv_create(model.handle, layer, max_tokens, C.byref(h)))
            _handle = h
        self.handle = _handle
        self.ctx._adopt(self)

    def info(self) -> tuple[int, int, int, bool]:
        """(rows held, heads, head_dim, has det data)."""
        n, h, d, has = C.c_uint64(), C.c_uint64(), C.c_uint64(), C.c_int32()
        self.ctx.check(self.ctx.lib.det_kv_info(self.handle, C.byref(n), C.byref(h), C.byref(d), C.byref(has)))
        return n.value, h.value, d.value, bool(has.value)

    def read_logical(self) -> tuple[np.ndarray, np.ndarray]:
        """Keys and values [heads][len][head_dim], oldest row first."""
        n, h, d, _ = self.info()
        k = np.empty((h, n, d), dtype=np.int32)
        v = np.empty((h, n, d), dtype=np.int32)
        self.ctx.check(self.ctx.lib.det_kv_read_logical(self.handle, _ptr(k), _ptr(v), k.size))
        return k, v

    def clone(self) -> "KvCache":
        h = C.c_void_p()
        self.ctx.check(self.ctx.lib.det_kv_clone(self.handle, C.byref(h)))
        return KvCache(self.model, self.layer, 0, _handle=h)

    def _release(self) -> None:
        if self.handle and self.ctx.handle:
            self.ctx.lib.det_kv_free(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self._release()
        except Exception:
            pass


def kv_commitment(caches) -> str | None:
    """build_det_kv_cache_commitment over the caches in order (None if one lacks det data)."""
    caches = list(caches)
    ctx = caches[0].ctx
    handles = (C.c_void_p * len(caches))(*[c.handle for c in caches])
    out = C.create_string_buffer(65)
    some = C.c_int32()
    ctx.check(ctx.lib.det_kv_commitment(C.cast(handles, C.c_void_p), len(caches), out, C.byref(some)))
    return out.value.decode() if some.value else None


class LayerOps:
    """The layer-level operators (det_kernels.rs API) of one model on device buffers."""

    def __init__(self, model: "Model"):
        self.model, self.ctx = model, model.ctx
        self.scratch = Scratch(model)

    def embed(self, ids, out) -> None:
        a = np.asarray(ids, dtype=np.uint32)
        self.ctx.check(self.ctx.lib.det_embed_tokens(self.model.handle, self.scratch.handle, _ptr(a), a.size,
                                                     _dptr(out)))

    def prefill_ple_inputs(self, layer: int, ids, inp, out) -> bool:
        a = np.asarray(ids, dtype=np.uint32)
        produced = C.c_int32()
        self.ctx.check(self.ctx.lib.det_prefill_ple_inputs(self.model.handle, self.scratch.handle, layer, _ptr(a),
                                                           a.size, _dptr(inp), _dptr(out), C.byref(produced)))
        return bool(produced.value)

    def decode_ple_input(self, token: int, inp, layer: int, out) -> bool:
        produced = C.c_int32()
        self.ctx.check(self.ctx.lib.det_decode_ple_input(self.model.handle, self.scratch.handle, int(token),
                                                         _dptr(inp), layer, _dptr(out), C.byref(produced)))
        return bool(produced.value)

    def layer_prefill(self, layer: int, xs, n: int, ple, donor: KvCache | None, cache: KvCache | None, out) -> None:
        self.ctx.check(self.ctx.lib.det_layer_prefill(self.model.handle, self.scratch.handle, layer, _dptr(xs), n,
                                                      _dptr(ple), donor.handle if donor else None,
                                                      cache.handle if cache else None, _dptr(out)))

    def layer_decode(self, layer: int, inp, ple, cache: KvCache | None, donor: KvCache | None, position: int,
                     out) -> None:
        self.ctx.check(self.ctx.lib.det_layer_decode(self.model.handle, self.scratch.handle, layer, _dptr(inp),
                                                     _dptr(ple), cache.handle if cache else None,
                                                     donor.handle if donor else None, position, _dptr(out)))

    def hidden_to_logits(self, hidden, out) -> None:
        self.ctx.check(self.ctx.lib.det_hidden_to_logits(self.model.handle, self.scratch.handle, _dptr(hidden),
                                                         _dptr(out)))


def decode_batch(sessions, tokens, flags: int = DET_COMMIT_ALL) -> list:
    """One decode step for each session (same model) in shared launches;
    results[i] is bit-identical to sessions[i].decode(tokens[i], flags)."""
    sessions = list(sessions)
    if not sessions:
        raise ValueError("decode_batch needs at least one session")
    toks = np.asarray(tokens, dtype=np.uint32)
    if toks.size != len(sessions):
        raise ValueError("one token per session")
    ctx = sessions[0].ctx
    handles = (C.c_void_p * len(sessions))(*[s.handle for s in sessions])
    res = (DecodeResult * len(sessions))()
    ctx.check(ctx.lib.det_session_decode_batch(C.cast(handles, C.c_void_p), len(sessions), _ptr(toks), flags,
                                               C.cast(res, C.c_void_p)))
    return list(res)


from . import synthetic  # noqa: E402,F401
