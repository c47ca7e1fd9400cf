"""ctypes loader for the CPU oracle (test infrastructure only).

The oracle restates the reference's deterministic path in C++ (see
oracle/oracle.h). Tests, the smoke check and bench.py's cpu_baseline leg use
it as the checker; nothing in the product imports it.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import pathlib
import subprocess

import numpy as np

REPO = pathlib.Path(__file__).resolve().parents[1]
ORACLE_DIR = REPO / "oracle"
ORACLE_SO = ORACLE_DIR / "build" / "liboracle.so"


class OrcTextConfig(C.Structure):
    """Mirror of orc_text_config (oracle/oracle.h)."""

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


def _opt(cfg: dict, out: C.Structure, key: str, field: str | None = None, conv=lambda v: v) -> None:
    field = field or key
    value = cfg.get(key)
    if value is not None:
        setattr(out, "has_" + field, 1)
        setattr(out, field, conv(value))


def oracle_config(config_json: dict) -> tuple[OrcTextConfig, object]:
    """Builds the raw config struct from a Gemma config.json dict.

    Follows the serde field set of GemmaTextConfigFile (gemma/io.rs:60-96);
    returns the struct and the array that owns the layer_types storage.
    """
    tc = config_json.get("text_config", config_json)
    out = OrcTextConfig()
    out.enable_moe_block = int(bool(tc["enable_moe_block"]))
    out.hidden_activation_is_gelu_pytorch_tanh = int(tc["hidden_activation"] == "gelu_pytorch_tanh")
    _opt(tc, out, "final_logit_softcapping", conv=float)
    _opt(tc, out, "global_head_dim", conv=int)
    out.head_dim = tc["head_dim"]
    out.hidden_size = tc["hidden_size"]
    _opt(tc, out, "hidden_size_per_layer_input", conv=int)
    types = (C.c_int32 * len(tc["layer_types"]))(*[int(t == "sliding_attention") for t in tc["layer_types"]])
    out.num_layer_types = len(tc["layer_types"])
    out.layer_types = C.cast(types, C.POINTER(C.c_int32))
    _opt(tc, out, "num_global_key_value_heads", conv=int)
    out.num_attention_heads = tc["num_attention_heads"]
    out.num_hidden_layers = tc["num_hidden_layers"]
    out.num_key_value_heads = tc["num_key_value_heads"]
    out.rms_norm_eps = float(np.float32(tc["rms_norm_eps"]))
    rp = tc.get("rope_parameters") or {}
    full = rp.get("full_attention") or {}
    sliding = rp.get("sliding_attention") or {}
    if full.get("partial_rotary_factor") is not None:
        out.has_full_partial_rotary_factor, out.full_partial_rotary_factor = 1, float(full["partial_rotary_factor"])
    if full.get("rope_theta") is not None:
        out.has_full_rope_theta, out.full_rope_theta = 1, float(full["rope_theta"])
    if sliding.get("rope_theta") is not None:
        out.has_sliding_rope_theta, out.sliding_rope_theta = 1, float(sliding["rope_theta"])
    if rp.get("rope_theta") is not None:
        out.has_rope_theta, out.rope_theta = 1, float(rp["rope_theta"])
    out.sliding_window = tc["sliding_window"]
    _opt(tc, out, "tie_word_embeddings", conv=int)
    out.vocab_size = tc["vocab_size"]
    _opt(tc, out, "vocab_size_per_layer_input", conv=int)
    _opt(tc, out, "attention_k_eq_v", conv=int)
    _opt(tc, out, "num_kv_shared_layers", conv=int)
    out.bidirectional_all = int(tc.get("use_bidirectional_attention") == "all")
    return out, types


def build_oracle(force: bool = False) -> pathlib.Path:
    if force or not ORACLE_SO.exists():
        subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return ORACLE_SO


_LIB = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        build_oracle()
        L = C.CDLL(str(ORACLE_SO))
        P = C.c_void_p
        i32p, i64p = C.POINTER(C.c_int32), C.POINTER(C.c_int64)
        L.orc_last_error.restype = C.c_char_p
        L.orc_scalar_last_error.restype = C.c_char_p
        for name, res, args in [
            ("orc_mac_bits", C.c_int64, [C.c_int64, C.c_int32, C.c_int32]),
            ("orc_acc_combine", C.c_int64, [C.c_int64, C.c_int64]),
            ("orc_add_sat", C.c_int32, [C.c_int32, C.c_int32]),
            ("orc_sub_sat", C.c_int32, [C.c_int32, C.c_int32]),
            ("orc_acc_add_sat", C.c_int64, [C.c_int64, C.c_int64]),
            ("orc_mul_sat", C.c_int32, [C.c_int32, C.c_int32]),
            ("orc_requantize", C.c_int32, [C.c_int64]),
            ("orc_rshift_round_ties_even", C.c_int, [C.c_int64, C.c_uint32, i64p]),
            ("orc_div_act", C.c_int, [C.c_int32, C.c_int32, i32p]),
            ("orc_div_acc", C.c_int, [C.c_int64, C.c_int64, i64p]),
            ("orc_div_acc_by_u32", C.c_int, [C.c_int64, C.c_uint32, i64p]),
            ("orc_acc_mul", C.c_int64, [C.c_int64, C.c_int64]),
            ("orc_inv_sqrt_acc", C.c_int, [C.c_int64, i32p]),
            ("orc_rms_norm_scale", C.c_int, [P, C.c_size_t, C.c_int64, i32p]),
            ("orc_rms_norm", C.c_int, [P, P, C.c_size_t, C.c_int64]),
            ("orc_value_rms_norm", C.c_int, [P, C.c_size_t, C.c_int64]),
            ("orc_attention_score", C.c_int, [P, P, C.c_size_t, i32p]),
            ("orc_attention_softmax_exp_term", C.c_int, [C.c_int32, C.c_int32, i64p]),
            ("orc_attention_softmax", C.c_int, [P, C.c_size_t, P]),
            ("orc_attention_weighted_sum", C.c_int, [P, P, C.c_size_t, C.c_size_t, P]),
            ("orc_tanh_act", C.c_int32, [C.c_int32]),
            ("orc_softcap_act", C.c_int, [C.c_int32, C.c_int32, i32p]),
            ("orc_gelu_pytorch_tanh_act", C.c_int32, [C.c_int32]),
            ("orc_nth_root_acc", C.c_int, [C.c_int64, C.c_uint32, i64p]),
            ("orc_rope_frequency_step", C.c_int, [C.c_int64, C.c_size_t, i64p]),
            ("orc_sin_cos_acc", None, [C.c_int64, i32p, i32p]),
            ("orc_rope_rotate_pairs", C.c_int, [P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int64, C.c_size_t]),
            ("orc_argmax_first", C.c_int, [P, C.c_size_t, C.POINTER(C.c_size_t)]),
            ("orc_f32_to_act", C.c_int, [C.c_float, i32p]),
            ("orc_f32_to_wgt", C.c_int, [C.c_float, i32p]),
            ("orc_f32_to_acc", C.c_int, [C.c_float, i64p]),
            ("orc_det_linear", C.c_int, [C.c_size_t, C.c_size_t, C.c_int, P, P, P, C.c_int]),
            ("orc_det_linear_acc_i64", C.c_int, [C.c_size_t, C.c_size_t, C.c_int, P, P, P]),
            ("orc_det_linear_slab", C.c_int, [C.c_size_t, C.c_size_t, C.c_size_t, C.c_int, P, P, P, C.c_int]),
            ("orc_attention_causal", C.c_int, [P, P, P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t,
                                               C.c_size_t, C.c_size_t, P, C.c_int]),
            ("orc_rope_inv_frequencies", C.c_int, [C.c_int64, C.c_size_t, C.c_size_t, P]),
            ("orc_commit_activation_rows", None, [P, C.c_size_t, C.c_size_t, C.c_char_p]),
            ("orc_commit_vector", None, [P, C.c_size_t, C.c_char_p]),
            ("orc_model_create", C.c_int, [C.POINTER(OrcTextConfig), C.POINTER(P)]),
            ("orc_model_set_tensor", C.c_int, [P, C.c_char_p, C.c_size_t, P, C.c_int, P, P]),
            ("orc_model_load_detwgt", C.c_int, [P, P, C.c_size_t]),
            ("orc_model_finalize", C.c_int, [P]),
            ("orc_model_free", None, [P]),
            ("orc_set_threads", None, [C.c_int]),
            ("orc_set_slab_group", None, [C.c_int]),
            ("orc_capture", C.c_int, [P, P, C.c_size_t, C.c_size_t, C.c_char_p, C.c_size_t]),
            ("orc_trace_capture", C.c_int, [P, P, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, C.c_char_p,
                                            C.c_size_t]),
            ("orc_session_prefill", C.c_int, [P, P, C.c_size_t, C.POINTER(P), P]),
            ("orc_session_decode", C.c_int, [P, C.c_uint32, P, P]),
            ("orc_session_clone", C.c_int, [P, P]),
            ("orc_session_free", None, [P]),
        ]:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


class OracleError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"oracle status {status}: {message}")
        self.status = status


def check(status: int, scalar: bool = False) -> None:
    if status != 0:
        msg = (lib().orc_scalar_last_error() if scalar else lib().orc_last_error()).decode()
        raise OracleError(status, msg)


def ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data)


class OracleModel:
    """A finalized oracle model (Gemma4TransformerModel in det mode)."""

    def __init__(self, config_json: dict):
        self._cfg, self._types = oracle_config(config_json)
        h = C.c_void_p()
        check(lib().orc_model_create(C.byref(self._cfg), C.byref(h)))
        self.handle = h
        self.config = config_json.get("text_config", config_json)

    def load_detwgt(self, data: bytes) -> "OracleModel":
        buf = np.frombuffer(data, dtype=np.uint8)
        check(lib().orc_model_load_detwgt(self.handle, ptr(buf), buf.size))
        return self

    def set_tensor(self, name: str, values: np.ndarray, width: int, row_scale: np.ndarray | None = None):
        dims = np.asarray(values.shape, dtype=np.uint64)
        values = np.ascontiguousarray(values)
        rs = None if row_scale is None else ptr(np.ascontiguousarray(row_scale, dtype=np.int32))
        check(lib().orc_model_set_tensor(self.handle, name.encode(), values.ndim, ptr(dims), width, ptr(values), rs))

    def finalize(self) -> "OracleModel":
        check(lib().orc_model_finalize(self.handle))
        return self

    def capture(self, prompt: list[int], decode_steps: int) -> dict:
        ids = np.asarray(prompt, dtype=np.uint32)
        cap = 1 << 20
        buf = C.create_string_buffer(cap + decode_steps * 512)
        check(lib().orc_capture(self.handle, ptr(ids), ids.size, decode_steps, buf, len(buf)))
        return json.loads(buf.value.decode())

    def trace_capture(self, prompt: list[int], decode_steps: int, prefill_width: int = 0,
                      decode_width: int = 0) -> dict:
        """Commitments of the routines' checkpoints (orc_trace_capture)."""
        ids = np.asarray(prompt, dtype=np.uint32)
        layers = int(self.config["num_hidden_layers"])
        n_ranges = -(-ids.size // max(prefill_width or ids.size, 1))
        cap = (1 << 16) + layers * (200 + 70 * n_ranges) + decode_steps * (400 + 200 * layers)
        buf = C.create_string_buffer(cap)
        check(lib().orc_trace_capture(self.handle, ptr(ids), ids.size, decode_steps, prefill_width, decode_width, buf,
                                      len(buf)))
        return json.loads(buf.value.decode())

    def session(self, prompt: list[int]) -> "OracleSession":
        """Prefills the prompt (pipeline::run_prefill_pass_with_mode) and returns the session."""
        return OracleSession(self, prompt)

    def __del__(self):
        h = getattr(self, "handle", None)
        if h and _LIB is not None:
            _LIB.orc_model_free(h)
            self.handle = None


class OracleSession:
    """One sequence on the oracle: prefill, then greedy decode steps."""

    def __init__(self, model: OracleModel, prompt: list[int]):
        self.model = model  # keeps the weights alive
        self.vocab = int(model.config["vocab_size"])
        self.hidden = int(model.config["hidden_size"])
        ids = np.asarray(prompt, dtype=np.uint32)
        self.logits = np.empty(self.vocab, dtype=np.int32)
        h = C.c_void_p()
        check(lib().orc_session_prefill(model.handle, ptr(ids), ids.size, C.byref(h), ptr(self.logits)))
        self.handle = h

    def next_token(self) -> int:
        return int(np.argmax(self.logits))  # argmax_first: numpy returns the first maximum

    def clone(self) -> "OracleSession":
        """An independent copy (caches, position, last logits)."""
        c = OracleSession.__new__(OracleSession)
        c.model, c.vocab, c.hidden = self.model, self.vocab, self.hidden
        c.logits = self.logits.copy()
        h = C.c_void_p()
        check(lib().orc_session_clone(self.handle, C.byref(h)))
        c.handle = h
        return c

    def decode(self, token: int) -> np.ndarray:
        """One decode step; returns the activation row (logits in self.logits)."""
        hidden = np.empty(self.hidden, dtype=np.int32)
        check(lib().orc_session_decode(self.handle, int(token), ptr(self.logits), ptr(hidden)))
        return hidden

    def __del__(self):
        h = getattr(self, "handle", None)
        if h and _LIB is not None:
            _LIB.orc_session_free(h)
            self.handle = None


def attention_causal(q, k, v, n_queries, n_rows, num_heads, num_kv_heads, head_dim, window, threads=1):
    """det_attention_prefill's items on seq-major q [nq][nh*hd], k/v [nrows][nkv*hd]."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.int32) for x in (q, k, v))
    out = np.zeros((n_queries, num_heads * head_dim), dtype=np.int32)
    check(lib().orc_attention_causal(ptr(q), ptr(k), ptr(v), n_queries, n_rows, num_heads, num_kv_heads, head_dim,
                                     window, ptr(out), threads))
    return out


def rope_inv_frequencies(base_acc: int, freq_base_dim: int, half: int) -> np.ndarray:
    out = np.empty(half, dtype=np.int64)
    check(lib().orc_rope_inv_frequencies(base_acc, freq_base_dim, half, ptr(out)))
    return out


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def set_slab_group(tokens: int) -> None:
    """Token rows per slab work item: 1 is the reference's schedule; larger
    groups read each weight row once per group (the same sums, faster for the
    long prompts of the E4B tests)."""
    lib().orc_set_slab_group(int(tokens))


def det_linear(weight: np.ndarray, act: np.ndarray, threads: int = 1) -> np.ndarray:
    w = np.ascontiguousarray(weight)
    width = {np.dtype(np.int16): 16, np.dtype(np.int32): 32}[w.dtype]
    a = np.ascontiguousarray(act, dtype=np.int32)
    out = np.empty(w.shape[0], dtype=np.int32)
    check(lib().orc_det_linear(w.shape[0], w.shape[1], width, ptr(w), ptr(a), ptr(out), threads))
    return out


def det_linear_slab(weight: np.ndarray, acts: np.ndarray, threads: int = 1) -> np.ndarray:
    w = np.ascontiguousarray(weight)
    width = {np.dtype(np.int16): 16, np.dtype(np.int32): 32}[w.dtype]
    a = np.ascontiguousarray(acts, dtype=np.int32)
    out = np.empty((a.shape[0], w.shape[0]), dtype=np.int32)
    check(lib().orc_det_linear_slab(a.shape[0], w.shape[0], w.shape[1], width, ptr(w), ptr(a), ptr(out), threads))
    return out


def det_linear_acc_i64(weight: np.ndarray, act: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(weight)
    width = {np.dtype(np.int16): 16, np.dtype(np.int32): 32}[w.dtype]
    a = np.ascontiguousarray(act, dtype=np.int32)
    out = np.empty(w.shape[0], dtype=np.int64)
    check(lib().orc_det_linear_acc_i64(w.shape[0], w.shape[1], width, ptr(w), ptr(a), ptr(out)))
    return out


def cpu_count() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
