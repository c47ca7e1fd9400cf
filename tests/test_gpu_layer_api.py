"""GPU parity of the layer-level operators (det_layer_prefill,
det_layer_decode, det_decode_ple_input, det_hidden_to_logits, KV handles).

The routines call these per layer (prefill_range/native/deterministic_tiles.rs
:69-199, decode_layer_range/native/tiles.rs:133-197). Here a host loop
restates the det_goldens capture protocol (src/runtime/det_goldens.rs:90-236)
on top of them, every call going through the C ABI, and must reproduce the
reference's goldens (tests/golden/det_commitment_goldens.det.json, both PLE
fixtures, one with a KV-sharing donor layer) and the oracle's capture of an
E4B-shaped model.
"""
import hashlib
import struct

import numpy as np
import pytest

import fixtures
import oracle_lib

pytestmark = pytest.mark.gpu
rd = pytest.importorskip("rasterdet")
from rasterdet import synthetic  # noqa: E402


@pytest.fixture(scope="module")
def ctx():
    c = rd.Context(0)
    yield c
    c.close()


def act_commitment(rows: np.ndarray) -> str:
    # build_det_activation_commitment (transformer_kernels.rs:1395-1430)
    rows = np.atleast_2d(rows).astype("<i4")
    h = hashlib.sha256(b"raster-det-num-act-v1" + struct.pack("<Q", rows.shape[0]))
    for r in rows:
        h.update(struct.pack("<Q", r.size) + r.tobytes())
    return h.hexdigest()


def vector_commitment(v: np.ndarray) -> str:
    # build_det_vector_commitment (transformer_kernels.rs:1432-1438)
    v = np.asarray(v).astype("<i4")
    return hashlib.sha256(b"raster-det-num-act-vector-v1" + struct.pack("<Q", v.size) + v.tobytes()).hexdigest()


def donor_of(tc: dict, layer: int):
    # kv_shared_layer_index (gemma/io.rs:165-190): the last layer before the
    # shared block with the same attention type
    shared = tc.get("num_kv_shared_layers") or 0
    first = tc["num_hidden_layers"] - shared
    if not shared or layer < first:
        return None
    return max(i for i in range(first) if tc["layer_types"][i] == tc["layer_types"][layer])


class LayerLoop:
    """det_goldens capture through the layer-level entry points."""

    def __init__(self, ctx, model, config, max_tokens):
        self.ctx, self.model, self.ops = ctx, model, rd.LayerOps(model)
        self.tc = config.get("text_config", config)
        self.H, self.L = self.tc["hidden_size"], self.tc["num_hidden_layers"]
        self.ple = self.tc.get("hidden_size_per_layer_input") or 0
        self.max_tokens = max_tokens

    def buf(self, rows, width):
        return self.ctx.empty((max(rows, 1), max(width, 1)))

    def ple_rows(self, ids, emb, n):
        out = []
        for layer in range(self.L):
            b = self.buf(n, self.ple)
            made = (self.ops.prefill_ple_inputs(layer, ids, emb, b) if n > 1
                    else self.ops.decode_ple_input(ids[0], emb, layer, b))
            out.append(b if made else None)
        return out

    def logits(self, hidden_row):
        out = self.ctx.empty(self.tc["vocab_size"])
        self.ops.hidden_to_logits(hidden_row, out)
        return out.numpy()

    def prefill(self, ids):
        n, H = len(ids), self.H
        emb = self.buf(n, H)
        self.ops.embed(ids, emb)
        ple = self.ple_rows(ids, emb, n)
        caches, x = [], self.buf(n, H)
        self.ctx.check(self.ctx.lib.det_memcpy_d2d(self.ctx.handle, rd.C.c_void_p(x.ptr), rd.C.c_void_p(emb.ptr),
                                                   n * H * 4))
        for layer in range(self.L):
            d = donor_of(self.tc, layer)
            cache = rd.KvCache(self.model, layer, self.max_tokens)
            self.ops.layer_prefill(layer, x, n, ple[layer], caches[d] if d is not None else None,
                                   None if d is not None else cache, x)
            caches.append(cache)
        hidden = x.numpy().reshape(n, H)
        last = self.ctx.to_device(np.ascontiguousarray(hidden[-1]))
        lg = self.logits(last)
        return caches, lg, {"embedding": act_commitment(emb.numpy().reshape(n, H)),
                            "final_hidden": act_commitment(hidden), "logits": vector_commitment(lg),
                            "kv": rd.kv_commitment(caches)}

    def decode(self, caches, token, position, per_layer=None):
        """One step on `caches` in place; per_layer collects (layer output,
        effective-cache commitment) with the untouched `original` caches."""
        emb = self.buf(1, self.H)
        self.ops.embed([token], emb)
        ple = self.ple_rows([token], emb, 1)
        x = self.ctx.to_device(emb.numpy().reshape(-1))
        for layer in range(self.L):
            d = donor_of(self.tc, layer)
            self.ops.layer_decode(layer, x, ple[layer], None if d is not None else caches[layer],
                                  caches[d] if d is not None else None, position, x)
            if per_layer is not None:
                original = per_layer["original"]
                eff = caches[:layer + 1] + original[layer + 1:]
                per_layer["layers"].append({"layer_output": act_commitment(x.numpy()),
                                            "kv": rd.kv_commitment(eff)})
        return x.numpy()

    def capture(self, ids, steps):
        caches, lg, pre = self.prefill(ids)
        out = {"prefill": pre}
        tok = int(np.argmax(lg))
        first = {"original": caches, "layers": []}
        copies = [c.clone() for c in caches]
        self.decode(copies, tok, len(ids), first)
        out["first_step_layers"] = first["layers"]
        out["decode_steps"], gen = [], []
        for i in range(steps):
            tok = int(np.argmax(lg))
            gen.append(tok)
            act = self.decode(caches, tok, len(ids) + i)
            lg = self.logits(self.ctx.to_device(act))
            out["decode_steps"].append({"token": tok, "activation": act_commitment(act),
                                        "logits": vector_commitment(lg), "kv": rd.kv_commitment(caches)})
        text = "[" + ",".join(map(str, gen)) + "]"
        out["end_to_end"] = {"generated_token_ids": gen,
                             "generated_token_ids_sha256": hashlib.sha256(text.encode()).hexdigest()}
        return out


@pytest.mark.parametrize("name", ["donor_ple", "no_donor_ple"])
def test_layer_loop_reproduces_reference_goldens(ctx, name):
    cfg, wgt, prompt, _ = fixtures.golden_fixture(name)
    steps = 16
    model = rd.Model(ctx, cfg).load_detwgt(wgt).finalize()
    got = LayerLoop(ctx, model, cfg, len(prompt) + steps + 1).capture(prompt, steps)
    exp = fixtures.golden_expected(name)
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"][:steps]


def test_layer_loop_e4b_shaped_matches_oracle(ctx):
    # int8 GEMM prefill, sliding ring wrapped (window 8 < 21 tokens)
    cfg = synthetic.e4b_config(layers=2, vocab=4096, sliding_window=8)
    om, gm = fixtures.load_both(cfg, synthetic.synthetic_model_fast(cfg, seed=7, scale_max=256), ctx,
                                threads=oracle_lib.cpu_count())
    prompt = list(range(3, 3 + 21))
    exp = om.capture(prompt, 5)
    got = LayerLoop(ctx, gm, cfg, len(prompt) + 6).capture(prompt, 5)
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"]
    assert got["end_to_end"] == exp["end_to_end"]


def test_kv_handles_read_logical_rows_and_reject_misuse(ctx):
    cfg = synthetic.e4b_config(layers=2, vocab=512, sliding_window=4)
    cfg["text_config"].update({"hidden_size": 128, "intermediate_size": 256, "head_dim": 32,
                               "num_attention_heads": 4, "num_key_value_heads": 2})
    gm = rd.Model(ctx, cfg)
    for name, v, s in fixtures.custom_model(cfg, seed=5):
        gm.set_tensor(name, v, s)
    gm.finalize()
    loop = LayerLoop(ctx, gm, cfg, 16)
    caches, _, _ = loop.prefill([1, 2, 3, 4, 5, 6])
    n0, heads, hd, has = caches[0].info()
    assert (n0, heads, hd, has) == (4, 2, 32, True)  # sliding window 4 keeps the last 4 rows
    assert caches[1].info()[0] == 6
    k0, v0 = caches[0].read_logical()
    k1, _ = caches[1].read_logical()
    assert k0.shape == (2, 4, 32) and k1.shape == (2, 6, 32)
    # one decode step appends one row; the ring drops its oldest
    loop.decode(caches, 7, 6)
    k0b, v0b = caches[0].read_logical()
    assert caches[0].info()[0] == 4
    assert np.array_equal(k0b[:, :3], k0[:, 1:]) and np.array_equal(v0b[:, :3], v0[:, 1:])
    k1b, _ = caches[1].read_logical()
    assert np.array_equal(k1b[:, :6], k1)
    empty = rd.KvCache(gm, 0, 8)
    assert empty.info()[3] is False
    assert rd.kv_commitment([empty, caches[1]]) is None  # a cache without det data
    x = ctx.empty((1, 128))
    with pytest.raises(rd.DetError):  # a layer-1 handle given to layer 0
        loop.ops.layer_decode(0, x, None, caches[1], None, 7, x)
    with pytest.raises(rd.DetError):  # neither a cache nor a donor
        loop.ops.layer_decode(0, x, None, None, None, 7, x)
    with pytest.raises(rd.DetError):
        rd.KvCache(gm, 2, 8)  # no such layer


def test_kv_handle_smaller_than_window_fails_closed(ctx):
    # a sliding-window cache created for fewer tokens than its window holds
    # max_tokens rows: a prefill or append past max_tokens must fail (the
    # reference's cache would still hold the last `window` rows) instead of
    # overwriting rows the window reads; a linear cache fails the same way,
    # and a ring sized at its window keeps taking tokens
    cfg = synthetic.e4b_config(layers=2, vocab=512, sliding_window=8)
    cfg["text_config"].update({"hidden_size": 128, "intermediate_size": 256, "head_dim": 32,
                               "num_attention_heads": 4, "num_key_value_heads": 2})
    gm = rd.Model(ctx, cfg)
    for name, v, s in fixtures.custom_model(cfg, seed=6):
        gm.set_tensor(name, v, s)
    gm.finalize()
    ops = rd.LayerOps(gm)
    x = ctx.to_device(np.zeros((6, 128), dtype=np.int32))
    small = rd.KvCache(gm, 0, 5)  # layer 0 is sliding (window 8), room for 5 tokens
    with pytest.raises(rd.DetError, match="KV cache capacity exceeded"):
        ops.layer_prefill(0, x, 6, None, None, small, x)
    small = rd.KvCache(gm, 0, 5)
    ops.layer_prefill(0, x, 5, None, None, small, x)
    assert small.info()[0] == 5
    row = ctx.to_device(np.zeros(128, dtype=np.int32))
    with pytest.raises(rd.DetError, match="KV cache capacity exceeded"):
        ops.layer_decode(0, row, None, small, None, 5, row)
    linear = rd.KvCache(gm, 1, 5)  # layer 1 is full attention
    ops.layer_prefill(1, x, 5, None, None, linear, x)
    with pytest.raises(rd.DetError, match="KV cache capacity exceeded"):
        ops.layer_decode(1, row, None, linear, None, 5, row)
    ring = rd.KvCache(gm, 0, 8)  # sized at the window: the trim keeps it going
    ops.layer_prefill(0, x, 5, None, None, ring, x)
    for pos in range(5, 12):
        ops.layer_decode(0, row, None, ring, None, pos, row)
    assert ring.info()[0] == 8
