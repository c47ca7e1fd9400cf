"""Fixture builders shared by the tests (data generation only).

* ``golden_fixture(name)`` rebuilds the two det_goldens fixtures exactly as the
  reference generates them (src/runtime/det_goldens.rs:288-514): same config,
  same LCG, same tensor order, converted with f32_to_wgt and encoded as a
  detwgt v2 artifact (det_num/artifact.rs:360-395).
* ``encode_detwgt`` is a plain restatement of that encoder.
"""
from __future__ import annotations

import json
import pathlib
import struct

import numpy as np

GOLDEN_DIR = pathlib.Path(__file__).resolve().parent / "golden"
MASK64 = (1 << 64) - 1


class FixtureRng:
    """det_goldens.rs:345-368. Weights are bucket/64 with bucket in [-16, 16]."""

    def __init__(self, seed: int):
        self.state = seed & MASK64

    def _bucket(self) -> int:
        self.state = (self.state * 6364136223846793005 + 1442695040888963407) & MASK64
        return ((self.state >> 33) % 33) - 16

    def weight_bits(self) -> int:
        # f32_to_wgt(bucket / 64.0): exact, = bucket * 1024.
        return self._bucket() * 1024

    def norm_bits(self) -> int:
        # f32_to_wgt(1.0 + (bucket / 64.0) / 4.0): exact, = 65536 + bucket * 256.
        return 65536 + self._bucket() * 256

    def weights(self, n: int) -> list[int]:
        return [self.weight_bits() for _ in range(n)]

    def norms(self, n: int) -> list[int]:
        return [self.norm_bits() for _ in range(n)]


def golden_config(donor: bool) -> dict:
    """det_goldens.rs:318-341."""
    return {
        "text_config": {
            "enable_moe_block": False,
            "head_dim": 2,
            "hidden_activation": "gelu_pytorch_tanh",
            "hidden_size": 4,
            "hidden_size_per_layer_input": 2,
            "layer_types": ["sliding_attention", "full_attention", "sliding_attention", "full_attention"],
            "num_attention_heads": 2,
            "num_hidden_layers": 4,
            "num_key_value_heads": 1,
            "num_kv_shared_layers": 1 if donor else 0,
            "rms_norm_eps": 0.000001,
            "sliding_window": 4,
            "tie_word_embeddings": False,
            "vocab_size": 9,
            "vocab_size_per_layer_input": 9,
        }
    }


def golden_tensors() -> list[tuple[str, list[int], list[int]]]:
    """det_goldens.rs:376-514 (tensor order fixes the LCG stream)."""
    H, HD, NH, NKV, L, FF, V, PLE = 4, 2, 2, 1, 4, 8, 9, 2
    rng = FixtureRng(0x5EED5EED5EED5EED)
    t: list[tuple[str, list[int], list[int]]] = []
    t.append(("model.language_model.embed_tokens.weight", [V, H], rng.weights(V * H)))
    for l in range(L):
        p = f"model.language_model.layers.{l}"
        t.append((f"{p}.self_attn.q_proj.weight", [NH * HD, H], rng.weights(NH * HD * H)))
        t.append((f"{p}.self_attn.k_proj.weight", [NKV * HD, H], rng.weights(NKV * HD * H)))
        t.append((f"{p}.self_attn.v_proj.weight", [NKV * HD, H], rng.weights(NKV * HD * H)))
        t.append((f"{p}.self_attn.o_proj.weight", [H, NH * HD], rng.weights(H * NH * HD)))
        t.append((f"{p}.self_attn.q_norm.weight", [HD], rng.norms(HD)))
        t.append((f"{p}.self_attn.k_norm.weight", [HD], rng.norms(HD)))
        for norm in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                     "post_feedforward_layernorm"):
            t.append((f"{p}.{norm}.weight", [H], rng.norms(H)))
        t.append((f"{p}.mlp.gate_proj.weight", [FF, H], rng.weights(FF * H)))
        t.append((f"{p}.mlp.up_proj.weight", [FF, H], rng.weights(FF * H)))
        t.append((f"{p}.mlp.down_proj.weight", [H, FF], rng.weights(H * FF)))
        t.append((f"{p}.per_layer_input_gate.weight", [PLE, H], rng.weights(PLE * H)))
        t.append((f"{p}.per_layer_projection.weight", [H, PLE], rng.weights(H * PLE)))
        t.append((f"{p}.post_per_layer_input_norm.weight", [H], rng.norms(H)))
    t.append(("model.language_model.embed_tokens_per_layer.weight", [V, L * PLE], rng.weights(V * L * PLE)))
    t.append(("model.language_model.per_layer_model_projection.weight", [L * PLE, H], rng.weights(L * PLE * H)))
    t.append(("model.language_model.per_layer_projection_norm.weight", [PLE], rng.norms(PLE)))
    t.append(("model.language_model.norm.weight", [H], rng.norms(H)))
    t.append(("model.language_model.lm_head.weight", [V, H], rng.weights(V * H)))
    return t


def encode_detwgt(tensors, force_i32: bool = False) -> bytes:
    """det_num/artifact.rs:360-395 (auto i16/i32 width, 64-byte aligned payloads)."""
    out = bytearray(b"DNWGTV0\0" + struct.pack("<IIQ", 2, 1, len(tensors)))
    for name, shape, bits in tensors:
        arr = np.asarray(bits, dtype=np.int64)
        fits16 = bool(arr.size == 0 or (arr.min() >= -32768 and arr.max() <= 32767))
        width = 32 if force_i32 or not fits16 else 16
        row = shape[-1] if shape else 1
        mass = int(np.abs(arr.reshape(-1, max(row, 1))).sum(axis=1).max()) if arr.size else 0
        nb = name.encode()
        count = int(np.prod(shape)) if shape else 1
        out += struct.pack("<I", len(nb)) + nb + struct.pack("<I", len(shape))
        out += b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<QIQQ", count, width, count * width // 8, mass)
        out += b"\0" * ((64 - len(out) % 64) % 64)
        out += arr.astype(np.int16 if width == 16 else np.int32).astype("<i" + str(width // 8)).tobytes()
    return bytes(out)


def golden_fixture(name: str):
    """Returns (config_json, detwgt bytes, prompt ids, decode steps)."""
    donor = {"donor_ple": True, "no_donor_ple": False}[name]
    # Prompt "w0 w1 w2 w3 w4 w5" through the WordLevel tokenizer of
    # det_goldens.rs:269-282 with no BOS/special tokens -> ids 0..5.
    return golden_config(donor), encode_detwgt(golden_tensors()), [0, 1, 2, 3, 4, 5], 64


def golden_expected(name: str) -> dict:
    return json.loads((GOLDEN_DIR / "det_commitment_goldens.det.json").read_text())[name]["det"]


def tiny_gemma_dev():
    d = GOLDEN_DIR / "tiny_gemma_dev"
    return json.loads((d / "config.json").read_text()), (d / "model.detwgt").read_bytes()


def custom_model(cfg: dict, seed: int, scale_max: int = 16, layer_scalars: bool = False):
    """Seeded int8 x scale tensors for a Gemma text config, honouring
    attention_k_eq_v (full layers without v_proj) and optional layer scalars.
    Returns a list of (name, values, row_scale)."""
    import sys
    sys.path.insert(0, str(GOLDEN_DIR.parents[1] / "raster-inference_amd"))
    from rasterdet import synthetic

    tc = cfg["text_config"]
    out = []
    for idx, (name, shape) in enumerate(synthetic.model_tensor_shapes(cfg)):
        if tc.get("attention_k_eq_v") and name.endswith("v_proj.weight"):
            layer = int(name.split(".layers.")[1].split(".")[0])
            if tc["layer_types"][layer] != "sliding_attention":
                continue
        ts = (seed * 1000003 + idx) & MASK64
        if len(shape) == 1:
            b = synthetic.hash_bytes(ts, shape[0]).astype(np.int32) % 33 - 16
            out.append((name, (65536 + b * 1024).astype(np.int32), None))
        else:
            q, s = synthetic.fast_int8_matrix(ts, shape[0], shape[1], scale_max)
            out.append((name, q, s))
    if layer_scalars:
        for l in range(tc["num_hidden_layers"]):
            out.append((f"model.language_model.layers.{l}.layer_scalar", np.array([65536 - 4096 * (l + 1)], dtype=np.int32), None))
    return out


def load_both(cfg, tensors, ctx, threads=8):
    """Builds the same model in the oracle and on the GPU."""
    import oracle_lib
    import rasterdet as rd

    om = oracle_lib.OracleModel(cfg)
    gm = rd.Model(ctx, cfg)
    for name, v, s in tensors:
        om.set_tensor(name, v, 8 if s is not None else {np.dtype(np.int16): 16}.get(np.asarray(v).dtype, 32), s)
        gm.set_tensor(name, v, s)
    oracle_lib.set_threads(threads)
    return om.finalize(), gm.finalize()
