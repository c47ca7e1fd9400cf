"""Seeded synthetic workloads of the det path (random-init weights, no downloads).

Weights are stored the way the MI355X path streams them: int8 q with a
per-row integer scale s (Wgt bits = q * s exactly). A detwgt v2 reader sees
the expanded bits; both views are the same matrix.

* ``tiny_model``   - Gemma-4-style decoder: 2 layers [sliding, full], hidden 64,
                     4/1 heads of 16, FF 128, vocab 512, untied, no PLE.
                     LCG buckets in [-16, 16] with s = 256; norm gains 1 + b/1024.
* ``e4b_model``    - E4B-shaped decoder: 42 layers alternating sliding/full,
                     hidden 2560, 8/2 heads of 256, FF 10240, vocab 262144.
* ``gemv_problem`` - int8 q uniform in [-127, 127], s uniform in [1, 256],
                     activation f32_to_act of a seeded normal.
"""
from __future__ import annotations

import numpy as np

MASK64 = (1 << 64) - 1


def splitmix64(seed: int, n: int) -> np.ndarray:
    """n outputs of splitmix64 starting from `seed` (uint64)."""
    out = np.empty(n, dtype=np.uint64)
    s = seed & MASK64
    for i in range(n):
        s = (s + 0x9E3779B97F4A7C15) & MASK64
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
        out[i] = z ^ (z >> 31)
    return out


def lcg_buckets(seed: int, n: int) -> np.ndarray:
    """Buckets in [-16, 16] from the 64-bit LCG stream (state*6364136223846793005 + 1442695040888963407)."""
    a, c = 6364136223846793005, 1442695040888963407
    # vectorised LCG jump: state_k = a^k s + c (a^k - 1)/(a - 1), computed by doubling
    states = np.empty(n, dtype=np.uint64)
    s = seed & MASK64
    block = 4096
    # step table for one block
    mults = np.empty(block, dtype=object)
    adds = np.empty(block, dtype=object)
    m, ad = 1, 0
    for k in range(block):
        m, ad = (m * a) & MASK64, (ad * a + c) & MASK64
        mults[k], adds[k] = m, ad
    mu = np.array([int(x) for x in mults], dtype=np.uint64)
    adu = np.array([int(x) for x in adds], dtype=np.uint64)
    i = 0
    while i < n:
        k = min(block, n - i)
        with np.errstate(over="ignore"):
            states[i:i + k] = mu[:k] * np.uint64(s) + adu[:k]
        s = int(states[i + k - 1])
        i += k
    return ((states >> np.uint64(33)) % np.uint64(33)).astype(np.int64) - 16


def f32_to_act(x: np.ndarray) -> np.ndarray:
    """Round-half-even of x * 2^16 with i32 saturation (exact for float32 inputs)."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64) * 65536.0  # exact: float32 * 2^16
    r = np.rint(x)  # half to even
    return np.clip(r, -2**31, 2**31 - 1).astype(np.int32)


def tiny_config() -> dict:
    return {"text_config": {
        "enable_moe_block": False, "head_dim": 16, "hidden_activation": "gelu_pytorch_tanh",
        "hidden_size": 64, "layer_types": ["sliding_attention", "full_attention"],
        "num_attention_heads": 4, "num_hidden_layers": 2, "num_key_value_heads": 1,
        "rms_norm_eps": 1e-6, "sliding_window": 128, "tie_word_embeddings": False, "vocab_size": 512,
    }}


def e4b_config(layers: int = 42, vocab: int = 262144, sliding_window: int = 512, ple: int = 0) -> dict:
    """E4B-shaped text config; ple > 0 adds per-layer inputs of that width
    (hidden_size_per_layer_input, over the same vocabulary)."""
    tc = {
        "enable_moe_block": False, "head_dim": 256, "hidden_activation": "gelu_pytorch_tanh",
        "hidden_size": 2560, "layer_types": [("sliding_attention" if l % 2 == 0 else "full_attention")
                                             for l in range(layers)],
        "num_attention_heads": 8, "num_hidden_layers": layers, "num_key_value_heads": 2,
        "rms_norm_eps": 1e-6, "sliding_window": sliding_window, "tie_word_embeddings": False,
        "vocab_size": vocab,
        "intermediate_size": 10240,
    }
    if ple:
        tc.update({"hidden_size_per_layer_input": ple, "vocab_size_per_layer_input": vocab})
    return {"text_config": tc}


def model_tensor_shapes(cfg: dict) -> list[tuple[str, tuple[int, ...]]]:
    """Tensor names/shapes of a Gemma-4 text decoder (gemma/io.rs naming), with
    the per-layer-input tensors when hidden_size_per_layer_input is set
    (gemma/io.rs:1183-1215, 1920-1940). Models without PLE keep their tensor order."""
    tc = cfg["text_config"]
    H, HD, NH, NKV = tc["hidden_size"], tc["head_dim"], tc["num_attention_heads"], tc["num_key_value_heads"]
    FF = tc.get("intermediate_size", 2 * H)
    V = tc["vocab_size"]
    L, P = tc["num_hidden_layers"], tc.get("hidden_size_per_layer_input") or 0
    out = [("model.language_model.embed_tokens.weight", (V, H))]
    for l in range(L):
        p = f"model.language_model.layers.{l}"
        out += [(f"{p}.self_attn.q_proj.weight", (NH * HD, H)), (f"{p}.self_attn.k_proj.weight", (NKV * HD, H)),
                (f"{p}.self_attn.v_proj.weight", (NKV * HD, H)), (f"{p}.self_attn.o_proj.weight", (H, NH * HD)),
                (f"{p}.self_attn.q_norm.weight", (HD,)), (f"{p}.self_attn.k_norm.weight", (HD,)),
                (f"{p}.input_layernorm.weight", (H,)), (f"{p}.post_attention_layernorm.weight", (H,)),
                (f"{p}.pre_feedforward_layernorm.weight", (H,)), (f"{p}.post_feedforward_layernorm.weight", (H,)),
                (f"{p}.mlp.gate_proj.weight", (FF, H)), (f"{p}.mlp.up_proj.weight", (FF, H)),
                (f"{p}.mlp.down_proj.weight", (H, FF))]
        if P:
            out += [(f"{p}.per_layer_input_gate.weight", (P, H)), (f"{p}.per_layer_projection.weight", (H, P)),
                    (f"{p}.post_per_layer_input_norm.weight", (H,))]
    if P:
        PV = tc.get("vocab_size_per_layer_input") or V
        out += [("model.language_model.embed_tokens_per_layer.weight", (PV, L * P)),
                ("model.language_model.per_layer_model_projection.weight", (L * P, H)),
                ("model.language_model.per_layer_projection_norm.weight", (P,))]
    out += [("model.language_model.norm.weight", (H,))]
    if not tc.get("tie_word_embeddings", True):
        out += [("model.language_model.lm_head.weight", (V, H))]
    return out


def tiny_model(seed: int = 0x5EED, head_dim: int = 16):
    """Config + tensors of the tiny parity model: list of (name, values, row_scale)."""
    cfg = tiny_config()
    cfg["text_config"]["intermediate_size"] = 128
    cfg["text_config"]["head_dim"] = head_dim
    tensors = []
    stream_seed = seed
    for name, shape in model_tensor_shapes(cfg):
        n = int(np.prod(shape))
        b = lcg_buckets(stream_seed, n)
        stream_seed = (stream_seed * 0x9E3779B97F4A7C15 + 1) & MASK64
        if len(shape) == 1:
            tensors.append((name, (65536 + b * 64).astype(np.int32), None))
        else:
            tensors.append((name, b.astype(np.int8).reshape(shape), np.full(shape[0], 256, dtype=np.int32)))
    return cfg, tensors


def tiny_prompt(n: int = 16, vocab: int = 512, seed: int = 0) -> list[int]:
    return [int(x % vocab) for x in splitmix64(seed, n)]


def random_int8_matrix(rng: np.random.Generator, rows: int, cols: int, scale_max: int = 256):
    q = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    s = rng.integers(1, scale_max + 1, size=rows, dtype=np.int32)
    return q, s


def gemv_problem(rows: int, cols: int, seed: int, scale_max: int = 256):
    rng = np.random.default_rng(seed)
    q, s = random_int8_matrix(rng, rows, cols, scale_max)
    act = f32_to_act(rng.standard_normal(cols).astype(np.float32))
    return q, s, act


def hash_bytes(seed: int, nbytes: int) -> np.ndarray:
    """nbytes pseudo-random bytes: splitmix64 finaliser over a counter (vectorised)."""
    n64 = (nbytes + 7) // 8
    x = np.arange(n64, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x += np.uint64((seed * 0x9E3779B97F4A7C15) & MASK64)
        x ^= x >> np.uint64(30)
        x *= np.uint64(0xBF58476D1CE4E5B9)
        x ^= x >> np.uint64(27)
        x *= np.uint64(0x94D049BB133111EB)
        x ^= x >> np.uint64(31)
    return x.view(np.uint8)[:nbytes]


def fast_int8_matrix(seed: int, rows: int, cols: int, scale_max: int):
    """q uniform-ish in [-127, 127] (byte % 255 - 127) and s in [1, scale_max], from counter hashes."""
    b = hash_bytes(seed, rows * cols)
    q = (b % np.uint8(255)).astype(np.int16) - 127
    q = q.astype(np.int8).reshape(rows, cols)
    sb = hash_bytes(seed ^ 0x5CA1E, rows * 4).view(np.uint32)
    s = (sb % np.uint32(scale_max)).astype(np.int32) + 1
    return q, s


def fast_i16_matrix(seed: int, rows: int, cols: int, lim: int = 4096, extremes: bool = True) -> np.ndarray:
    """Wgt bits uniform in [-lim, lim] from counter hashes (int16; with
    gcd 1 and values past 127 they do not factor into int8 x scale). With
    `extremes`, every 7th row holds 32767 and every 11th row -32768 at a
    hashed column, never both in one row (rows that need the negated or the
    plain two-digit form)."""
    b = hash_bytes(seed, rows * cols * 2).view(np.uint16).astype(np.int32)
    w = (b % (2 * lim + 1) - lim).astype(np.int16).reshape(rows, cols)
    w[:, 0] = 1
    if extremes and cols > 1:
        c = hash_bytes(seed ^ 0xE7, rows * 4).view(np.uint32) % np.uint32(cols - 1) + 1
        r = np.arange(rows)
        hi = r % 7 == 0
        lo = (r % 11 == 3) & ~hi
        w[r[hi], c[hi]] = 32767
        w[r[lo], c[lo]] = -32768
    return w


def synthetic_model_i16(cfg: dict, seed: int, lim: int = 4096):
    """The model of synthetic_model_fast with i16 Wgt bits that do not
    factor into int8 x scale (every matrix from fast_i16_matrix)."""
    for idx, (name, shape) in enumerate(model_tensor_shapes(cfg)):
        ts = (seed * 1000003 + idx) & MASK64
        if len(shape) == 1:
            b = hash_bytes(ts, shape[0]).astype(np.int32) % 33 - 16
            yield name, (65536 + b * 1024).astype(np.int32), None
        else:
            try:
                from . import synthetic_i16  # native generator (same values)
                yield name, synthetic_i16(ts, shape[0], shape[1], lim), None
            except RuntimeError:
                yield name, fast_i16_matrix(ts, shape[0], shape[1], lim), None


def synthetic_model_fast(cfg: dict, seed: int, scale_max: int = 16):
    """Like synthetic_model but with counter-hash weights (fast enough for E4B scale)."""
    for idx, (name, shape) in enumerate(model_tensor_shapes(cfg)):
        ts = (seed * 1000003 + idx) & MASK64
        if len(shape) == 1:
            b = hash_bytes(ts, shape[0]).astype(np.int32) % 33 - 16
            yield name, (65536 + b * 1024).astype(np.int32), None
        else:
            try:
                from . import synthetic_int8  # native generator (same values)
                q, s = synthetic_int8(ts, shape[0], shape[1], scale_max)
            except RuntimeError:
                q, s = fast_int8_matrix(ts, shape[0], shape[1], scale_max)
            yield name, q, s


def synthetic_model(cfg: dict, seed: int, scale_max: int = 16):
    """Random int8 x scale weights for any config (used for the E4B shape).

    Matrices: q uniform in [-127, 127], s uniform in [1, scale_max]; norm
    gains 1 + u/64 with u uniform in [-16, 16]. Generates lazily, one tensor
    at a time, so a 4.5 GB model never needs a second host copy.
    """
    rng = np.random.default_rng(seed)
    for name, shape in model_tensor_shapes(cfg):
        if len(shape) == 1:
            yield name, (65536 + rng.integers(-16, 17, size=shape) * 1024).astype(np.int32), None
        else:
            q, s = random_int8_matrix(rng, shape[0], shape[1], scale_max)
            yield name, q, s
