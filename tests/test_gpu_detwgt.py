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
