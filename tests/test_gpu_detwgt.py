"""GPU loader of detwgt artifacts (det_model_load_detwgt): a model loaded
from a detwgt-q8 artifact computes exactly what the same weights give from
detwgt v2 or from det_model_set_tensor, and malformed q8 files are rejected
fail-closed."""
import struct

import numpy as np
import pytest

import fixtures

pytestmark = pytest.mark.gpu
rd = pytest.importorskip("rasterdet")
from rasterdet import detwgt, synthetic  # noqa: E402


@pytest.fixture(scope="module")
def ctx():
    c = rd.Context(0)
    yield c
    c.close()


def test_q8_tiny_gemma_dev_captures_equal_v2(ctx):
    cfg, blob = fixtures.tiny_gemma_dev()
    q8 = detwgt.encode_q8(detwgt.parse(blob))
    prompt = [9, 10, 11, 11, 6, 3, 5, 14, 15, 8, 10, 5, 3, 4, 5, 6, 7, 4, 8]
    a = rd.Model(ctx, cfg).load_detwgt(blob).finalize().capture(prompt, 4)
    b = rd.Model(ctx, cfg).load_detwgt(q8).finalize().capture(prompt, 4)
    assert a == b


def test_q8_e4b_shaped_layers_equal_set_tensor(ctx):
    cfg = synthetic.e4b_config(layers=2, vocab=2048, sliding_window=8)
    tensors = list(synthetic.synthetic_model_fast(cfg, seed=23))
    art = detwgt.encode_q8([
        detwgt.Tensor(name, tuple(v.shape), q=v, scale=s) if s is not None
        else detwgt.Tensor(name, tuple(v.shape), bits=v) for name, v, s in tensors])
    direct = rd.Model(ctx, cfg)
    for name, v, s in tensors:
        direct.set_tensor(name, v, s)
    direct.finalize()
    loaded = rd.Model(ctx, cfg).load_detwgt(art).finalize()
    prompt = list(range(40, 53))
    assert loaded.capture(prompt, 3) == direct.capture(prompt, 3)


def bad_artifacts():
    t = [detwgt.Tensor("model.language_model.norm.weight", (4,), bits=np.full(4, 65536, np.int32)),
         detwgt.Tensor("m", (2, 3), q=np.array([[1, -2, 3], [4, 5, -6]], np.int8), scale=np.array([3, 7], np.int32))]
    good = detwgt.encode_q8(t)
    yield "magic", b"DNWGTQ9\0" + good[8:]
    yield "version", good[:8] + struct.pack("<I", 2) + good[12:]
    yield "trailing", good + b"\0"
    yield "truncated", good[:-1]
    patched = bytearray(good)
    patched[-9] = 1  # the alignment padding byte just before the row scales
    yield "padding", bytes(patched)
    big = bytearray(detwgt.encode_q8([detwgt.Tensor("x", (1, 2), q=np.array([[127, 1]], np.int8),
                                                    scale=np.array([1], np.int32))]))
    big[-4:] = struct.pack("<i", 2**25)
    yield "q*s range", bytes(big)


@pytest.mark.parametrize("case,data", list(bad_artifacts()), ids=[c[0] for c in bad_artifacts()])
def test_q8_loader_fails_closed(ctx, case, data):
    with pytest.raises(ValueError):
        detwgt.parse(data)  # the Python parser rejects it too
    cfg, _ = fixtures.tiny_gemma_dev()
    with pytest.raises(rd.DetError) as e:
        rd.Model(ctx, cfg).load_detwgt(data)
    assert e.value.status == 1


def v2_record(name: bytes, shape, width: int, payload_len: int, mass: int, payload: bytes = b"") -> bytes:
    """One detwgt v2 record (DETWGT_V2_FORMAT.md): name, rank, dims, element
    count, width tag, payload length, max row mass, then the 64-byte aligned
    payload (alignment counted from the start of the artifact)."""
    out = struct.pack("<I", len(name)) + name + struct.pack("<I", len(shape))
    count = 1
    for d in shape:
        out += struct.pack("<Q", d)
        count = (count * d) & ((1 << 64) - 1)
    return out + struct.pack("<QIQQ", count, width, payload_len, mass) + payload


def bad_v2_artifacts():
    t = [detwgt.Tensor("model.language_model.norm.weight", (4,), bits=np.full(4, 65536, np.int32)),
         detwgt.Tensor("m", (2, 3), bits=np.array([[1, -2, 3], [4, 5, -6]], np.int32))]
    good = detwgt.encode_v2(t)
    assert len(detwgt.parse(good)) == 2
    yield "version 1", good[:8] + struct.pack("<I", 1) + good[12:]
    yield "spec version 2", good[:12] + struct.pack("<I", 2) + good[16:]
    yield "trailing", good + b"\0"
    yield "truncated", good[:-2]
    padded = bytearray(good)
    padded[-24 - 1] = 7  # last alignment byte before the final i32 payload
    yield "padding", bytes(padded)
    head = b"DNWGTV0\0" + struct.pack("<IIQ", 2, 1, 1)
    heavy = head + v2_record(b"m", (1, 2), 32, 8, 1 << 31)
    heavy += b"\0" * (-len(heavy) % 64) + struct.pack("<ii", 1 << 30, 1 << 30)
    yield "row mass", heavy
    # 2^31 x 2^31 elements of width 32: the byte count 2^64 wraps to 0 in u64
    yield "payload byte count overflow", head + v2_record(b"w", (1 << 31, 1 << 31), 32, 0, 0)
    # a rank the artifact cannot hold (no allocation for 2^32 - 1 dimensions)
    yield "rank past the end", head + struct.pack("<I", 1) + b"w" + struct.pack("<I", 0xFFFFFFFF)


@pytest.mark.parametrize("case,data", list(bad_v2_artifacts()), ids=[c[0] for c in bad_v2_artifacts()])
def test_v2_loader_fails_closed(ctx, case, data):
    # the product's reader rejects what DetNumTensorReader::load_artifact
    # rejects (gemma/io.rs:224-387), with a status instead of a crash
    cfg, _ = fixtures.tiny_gemma_dev()
    with pytest.raises(rd.DetError) as e:
        rd.Model(ctx, cfg).load_detwgt(data)
    assert e.value.status == 1, str(e.value)
    if case == "payload byte count overflow":
        assert "payload byte count overflowed" in str(e.value)


def test_rope_base_i64_max_is_a_contract_violation(ctx):
    # rope theta >= 2^31 saturates to i64::MAX; the reference's nth_root_acc
    # overflows at the first rotation of a position > 0 (ops.rs:578). Position
    # 0 is the identity and never reaches it.
    x = ctx.to_device(np.arange(2 * 16, dtype=np.int32).reshape(2, 16))
    ctx.rope_rotate_pairs(x, 1, 1, 16, 16, 16, (1 << 63) - 1, 0, 0)  # position 0 only
    with pytest.raises(rd.DetError) as e:
        ctx.rope_rotate_pairs(x, 2, 1, 16, 16, 16, (1 << 63) - 1, 0, 1)
    assert e.value.status == 2
    cfg = synthetic.tiny_model()[0]
    cfg["text_config"]["rope_parameters"] = {"sliding_attention": {"rope_theta": 3.0e9}}
    gm = rd.Model(ctx, cfg)
    for name, v, s in synthetic.tiny_model()[1]:
        gm.set_tensor(name, v, s)
    gm.finalize()
    sess = gm.session(8)
    tok = sess.prefill([5]).next_token  # one token: position 0 only
    with pytest.raises(rd.DetError) as e:
        sess.decode(tok)
    assert e.value.status == 2
    with pytest.raises(rd.DetError) as e:
        gm.session(8).prefill([5, 6])
    assert e.value.status == 2
