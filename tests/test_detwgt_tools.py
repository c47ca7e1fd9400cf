"""Weight-format tooling (rasterdet.detwgt): the detwgt v2 writer and
safetensors converter against the reference's own artifacts and converter
tests, and the int8 variant (detwgt-q8) round trip and fail-closed parser."""
import json
import pathlib
import struct

import numpy as np
import pytest

from rasterdet import detwgt

TINY = pathlib.Path(__file__).resolve().parent / "golden" / "tiny_gemma_dev"


def safetensors_bytes(tensors) -> bytes:
    """A minimal .safetensors file: (name, dtype, shape, float values)."""
    header, blobs, off = {}, [], 0
    for name, dtype, shape, values in tensors:
        a = np.asarray(values, dtype=np.float32)
        if dtype == "BF16":
            raw = (a.view(np.uint32) >> 16).astype("<u2").tobytes()
        elif dtype == "F16":
            raw = a.astype("<f2").tobytes()
        else:
            raw = a.astype("<f4").tobytes()
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + b"".join(blobs)


def test_v2_writer_reproduces_the_reference_artifact():
    # tiny-gemma-dev/model.detwgt was written by the reference encoder
    # (tools/tiny-gemma-dev/main.rs:537-555 -> encode_det_wgt_artifact)
    ref = (TINY / "model.detwgt").read_bytes()
    assert detwgt.encode_v2(detwgt.parse(ref, verify_mass=True)) == ref


def test_converter_matches_the_reference_artifact_in_sorted_order():
    conv = detwgt.parse(detwgt.convert_safetensors((TINY / "model.safetensors").read_bytes()), verify_mass=True)
    ref = sorted(detwgt.parse((TINY / "model.detwgt").read_bytes()), key=lambda t: t.name)
    assert [t.name for t in conv] == [t.name for t in ref]
    for a, b in zip(conv, ref):
        assert a.shape == b.shape and a.width == b.width and np.array_equal(a.values(), b.values())


def test_converter_known_answers():
    # converter tests (tools/gemma-det-num-wgt-converter/main.rs:605-811)
    out = detwgt.parse(detwgt.convert_safetensors(safetensors_bytes([
        ("model.language_model.embed_tokens.weight", "BF16", (2, 2), [1.5, -2.0, 3.25, 4.5]),
        ("model.language_model.norm.weight", "F16", (2,), [0.5, 1.0])])), verify_mass=True)
    assert [t.name for t in out] == ["model.language_model.embed_tokens.weight", "model.language_model.norm.weight"]
    assert out[0].values().ravel().tolist() == [98304, -131072, 212992, 294912]
    assert detwgt.max_row_mass(out[0].shape, out[0].values()) == 507904
    assert out[1].values().tolist() == [32768, 65536]
    sat = detwgt.parse(detwgt.convert_safetensors(safetensors_bytes([
        ("tensor", "F32", (2, 2), [40000.0, 0.0, -3.5 / 65536.0, 3.5 / 65536.0])])))
    assert sat[0].values().ravel().tolist() == [2**31 - 1, 0, -4, 4]
    with pytest.raises(ValueError, match="overflow bound"):
        detwgt.convert_safetensors(safetensors_bytes([("tensor", "F32", (2, 2), [-40000.0, 0.0, 0.0, 0.0])]))
    norm = detwgt.parse(detwgt.convert_safetensors(safetensors_bytes([("model.norm.weight", "F32", (2,),
                                                                          [20000.0, 20000.0])])))
    assert detwgt.max_row_mass(norm[0].shape, norm[0].values()) == 2 * 20000 * 65536
    with pytest.raises(ValueError, match="non-finite"):
        detwgt.convert_safetensors(safetensors_bytes([("t", "F32", (1,), [float("inf")])]))


def test_i16_width_rule():
    small = detwgt.Tensor("a", (2, 2), bits=np.array([[1, -32768], [32767, 0]], np.int32))
    big = detwgt.Tensor("b", (2, 2), bits=np.array([[1, -32769], [0, 0]], np.int32))
    out = detwgt.parse(detwgt.encode_v2([small, big]))
    assert [t.width for t in out] == [16, 32]
    assert [t.width for t in detwgt.parse(detwgt.encode_v2([small], force_i32=True))] == [32]


def test_int8_factorization():
    w = np.array([[6, -12, 0, 762], [0, 0, 0, 0], [3, 5, 7, 11]], dtype=np.int64)
    q, s = detwgt.factor_int8(w)
    assert s.tolist() == [6, 1, 1] and np.array_equal(q.astype(np.int64) * s[:, None], w)
    assert detwgt.factor_int8(np.array([[1, 128]])) is None      # gcd 1, 128 does not fit
    assert detwgt.factor_int8(np.array([[-128, 2]])).__class__ is tuple


def test_q8_round_trip_of_the_tiny_model():
    ref = detwgt.parse((TINY / "model.detwgt").read_bytes())
    q8 = detwgt.encode_q8(ref)
    out = detwgt.parse(q8, verify_mass=True)
    assert [t.name for t in out] == [t.name for t in ref]
    assert all(np.array_equal(a.values(), b.values()) for a, b in zip(out, ref))
    assert all((t.width == 8) == (len(t.shape) == 2) for t in out)  # every tiny matrix factors
    assert detwgt.encode_q8(out) == q8


def corrupt_cases():
    t = [detwgt.Tensor("m", (2, 3), q=np.array([[1, -2, 3], [4, 5, -6]], np.int8), scale=np.array([3, 7], np.int32)),
         detwgt.Tensor("v", (3,), bits=np.array([1, 2, 3], np.int32))]
    good = detwgt.encode_q8(t)
    yield "ok", good, None
    yield "magic", b"DNWGTQ9\0" + good[8:], "magic"
    yield "version", good[:8] + struct.pack("<I", 2) + good[12:], "version"
    yield "trailing", good + b"\0", "trailing"
    yield "truncated", good[:-1], "ended unexpectedly"
    # name 'm' record: first padding byte follows the scale count
    hdr = 24 + 4 + 1 + 4 + 16 + 8 + 4 + 8 + 8
    yield "scale count", good[:hdr] + struct.pack("<Q", 3) + good[hdr + 8:], "scale count"
    yield "padding", good[:hdr + 8] + b"\1" + good[hdr + 9:], "padding"
    dup = detwgt.encode_q8([t[0], t[0]])
    yield "duplicate", dup, "duplicate"
    w8v = bytearray(detwgt.encode_q8([t[1]]))
    off = 24 + 4 + 1 + 4 + 8 + 8
    w8v[off:off + 4] = struct.pack("<I", 8)
    yield "width 8 vector", bytes(w8v), "element width"
    # a scale patched so that q * s leaves i32 (the writer refuses to write it)
    big = bytearray(detwgt.encode_q8([detwgt.Tensor("x", (1, 2), q=np.array([[127, 1]], np.int8),
                                                    scale=np.array([1], np.int32))]))
    big[-4:] = struct.pack("<i", 2**25)
    yield "q*s range", bytes(big), "outside i32"


@pytest.mark.parametrize("case,data,err", list(corrupt_cases()), ids=[c[0] for c in corrupt_cases()])
def test_q8_parser_fails_closed(case, data, err):
    if err is None:
        assert len(detwgt.parse(data)) == 2
    else:
        with pytest.raises(ValueError, match=err):
            detwgt.parse(data)


def test_row_mass_bound_applies_to_matrices_only():
    with pytest.raises(ValueError, match="overflow bound"):
        detwgt.encode_q8([detwgt.Tensor("m", (1, 2), bits=np.array([[2**31 - 1, 1]], np.int64))])
    assert detwgt.parse(detwgt.encode_v2([detwgt.Tensor("v", (2,), bits=np.array([2**31 - 1, 2**31 - 1]))]))
