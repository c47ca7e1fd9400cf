"""detwgt weight artifacts: writer, converter and audit.

* detwgt v2 (the reference's format; encoder det_num/artifact.rs:77-206,
  converter tools/gemma-det-num-wgt-converter/main.rs:218-390): canonical
  Q16.16 Wgt bits stored as i16 when every value of a tensor fits, else i32,
  64-byte aligned payloads, per-tensor max row mass with the overflow bound
  sum_i |w| < 2^31 enforced for rank >= 2 tensors.
* detwgt-q8: the same record layout under the magic ``DNWGTQ8\\0`` (format
  version 1), where a rank >= 2 tensor may also be stored as int8 q with one
  i32 scale per last-dimension row (W = q * s exactly, the form the GPU
  kernels consume). Its record adds ``scale_count`` (u64, = rows) after
  ``max_row_mass`` for width 8; the int8 payload and the scales each start at
  a 64-byte aligned offset. v2 loaders reject it by magic; libdetgpu's loader
  (det_model_load_detwgt) reads both.

``python -m rasterdet.detwgt convert model.safetensors out.detwgt [--int8]``
converts fp weights like the reference converter (sorted tensor names,
round-half-even f32 -> Q16.16, the same width rule); ``audit`` prints and
re-checks an artifact.
"""
from __future__ import annotations

import json
import math
import struct
import sys
from dataclasses import dataclass

import numpy as np

MAGIC_V2 = b"DNWGTV0\0"
MAGIC_Q8 = b"DNWGTQ8\0"
FORMAT_V2, FORMAT_Q8, SPEC_VERSION = 2, 1, 1
ALIGN = 64
ROW_MASS_LIMIT = 1 << 31


@dataclass
class Tensor:
    """One artifact tensor: canonical Wgt bits, or int8 q with row scales."""
    name: str
    shape: tuple[int, ...]
    bits: np.ndarray | None = None   # int32 canonical values (widths 16/32)
    q: np.ndarray | None = None      # int8 (width 8)
    scale: np.ndarray | None = None  # int32 per row (width 8)
    width: int = 32

    def values(self) -> np.ndarray:
        """Canonical Wgt bits (int64 to hold q * s before the range check)."""
        if self.q is not None:
            rows = self.q.reshape(-1, self.shape[-1]).astype(np.int64)
            return (rows * self.scale.astype(np.int64)[:, None]).reshape(self.shape)
        return self.bits.astype(np.int64).reshape(self.shape)


def f32_to_wgt(x: np.ndarray) -> np.ndarray:
    """f32_to_wgt (det_num/convert.rs:77-92): round half to even of x * 2^16,
    saturated to i32 (x * 2^16 is exact in float64 for every float32)."""
    x = np.asarray(x, dtype=np.float32)
    if not np.isfinite(x).all():
        raise ValueError("non-finite source values are not supported")
    r = np.rint(x.astype(np.float64) * 65536.0)
    return np.clip(r, -2**31, 2**31 - 1).astype(np.int32)


def max_row_mass(shape, values: np.ndarray) -> int:
    """max_r sum_i |w[r][i]| over last-dimension rows (artifact.rs max_row_mass)."""
    rows = np.abs(np.asarray(values, dtype=np.int64)).reshape(-1, max(shape[-1] if shape else 1, 1))
    return int(rows.sum(axis=1).max(initial=0)) if rows.size else 0


def _check_bound(t: Tensor, mass: int) -> None:
    if len(t.shape) >= 2 and mass >= ROW_MASS_LIMIT:
        raise ValueError(f"tensor `{t.name}` has row mass {mass}, violating the overflow bound "
                         f"(must be < {ROW_MASS_LIMIT})")


def _pad(buf: bytearray) -> None:
    buf.extend(b"\0" * ((-len(buf)) % ALIGN))


def _header(buf: bytearray, t: Tensor, width: int, mass: int) -> None:
    name = t.name.encode()
    count = int(np.prod(t.shape, dtype=np.uint64)) if t.shape else 1
    buf += struct.pack("<I", len(name)) + name + struct.pack("<I", len(t.shape))
    for d in t.shape:
        buf += struct.pack("<Q", d)
    buf += struct.pack("<QIQQ", count, width, count * width // 8, mass)


def encode_v2(tensors: list[Tensor], force_i32: bool = False) -> bytes:
    """A detwgt v2 artifact (encode_det_wgt_artifact_with_widths)."""
    buf = bytearray(MAGIC_V2 + struct.pack("<IIQ", FORMAT_V2, SPEC_VERSION, len(tensors)))
    for t in tensors:
        v = t.values()
        if v.min(initial=0) < -2**31 or v.max(initial=0) > 2**31 - 1:
            raise ValueError(f"tensor `{t.name}` has values outside i32")
        mass = max_row_mass(t.shape, v)
        _check_bound(t, mass)
        width = 32 if force_i32 or v.min(initial=0) < -32768 or v.max(initial=0) > 32767 else 16
        _header(buf, t, width, mass)
        _pad(buf)
        buf += v.astype("<i2" if width == 16 else "<i4").tobytes()
    return bytes(buf)


def factor_int8(values: np.ndarray) -> tuple[np.ndarray, np.ndarray] | None:
    """Exact int8 x row-scale form of a matrix: s_r = gcd of row r's |w|
    (1 for a zero row), q = w / s_r, when every q fits int8 (the largest
    scale that divides a row gives its smallest q, so no other scale fits if
    this one does not)."""
    rows = np.asarray(values, dtype=np.int64).reshape(-1, values.shape[-1])
    g = np.gcd.reduce(np.abs(rows), axis=1)
    g[g == 0] = 1
    q = rows // g[:, None]
    if q.min(initial=0) < -128 or q.max(initial=0) > 127 or g.max(initial=1) > 2**31 - 1:
        return None
    return q.astype(np.int8).reshape(values.shape), g.astype(np.int32)


def encode_q8(tensors: list[Tensor], allow_int8: bool = True) -> bytes:
    """A detwgt-q8 artifact: rank >= 2 tensors given as (q, scale), or whose
    values factor exactly, are stored at width 8; the rest as in v2."""
    buf = bytearray(MAGIC_Q8 + struct.pack("<IIQ", FORMAT_Q8, SPEC_VERSION, len(tensors)))
    for t in tensors:
        v = t.values()
        if v.min(initial=0) < -2**31 or v.max(initial=0) > 2**31 - 1:
            raise ValueError(f"tensor `{t.name}` has values outside i32")
        mass = max_row_mass(t.shape, v)
        _check_bound(t, mass)
        form = None
        if allow_int8 and len(t.shape) >= 2:
            form = (t.q, t.scale) if t.q is not None else factor_int8(v)
        if form is not None:
            q, s = form
            _header(buf, t, 8, mass)
            buf += struct.pack("<Q", s.size)
            _pad(buf)
            buf += np.ascontiguousarray(q, dtype=np.int8).tobytes()
            _pad(buf)
            buf += np.ascontiguousarray(s, dtype="<i4").tobytes()
            continue
        width = 32 if v.min(initial=0) < -32768 or v.max(initial=0) > 32767 else 16
        _header(buf, t, width, mass)
        _pad(buf)
        buf += v.astype("<i2" if width == 16 else "<i4").tobytes()
    return bytes(buf)


def parse(data: bytes, verify_mass: bool = False) -> list[Tensor]:
    """Parses a v2 or q8 artifact with the fail-closed checks of
    DetNumTensorReader::load_artifact (gemma/io.rs:224-387), extended to
    width 8 for q8. verify_mass also requires each max_row_mass field to equal
    the recomputed value (the reference re-checks only the bound)."""
    cur = 0

    def take(n: int) -> bytes:
        nonlocal cur
        if n > len(data) - cur:
            raise ValueError("artifact ended unexpectedly")
        b = data[cur:cur + n]
        cur += n
        return b

    def u32() -> int:
        return struct.unpack("<I", take(4))[0]

    def u64() -> int:
        return struct.unpack("<Q", take(8))[0]

    def pad(name: str) -> None:
        p = take((-cur) % ALIGN)
        if any(p):
            raise ValueError(f"tensor `{name}` has non-zero payload alignment padding")

    magic = take(8)
    if magic not in (MAGIC_V2, MAGIC_Q8):
        raise ValueError("unsupported deterministic artifact magic")
    q8 = magic == MAGIC_Q8
    if u32() != (FORMAT_Q8 if q8 else FORMAT_V2):
        raise ValueError("unsupported deterministic artifact format version")
    if u32() != SPEC_VERSION:
        raise ValueError("unsupported deterministic artifact det_num spec version; expected 1")
    out, seen = [], set()
    for _ in range(u64()):
        name = take(u32()).decode()
        shape = tuple(u64() for _ in range(u32()))
        count = math.prod(shape) if shape else 1
        if u64() != count:
            raise ValueError(f"tensor `{name}` element count mismatch")
        width = u32()
        if width not in ((8, 16, 32) if q8 else (16, 32)) or (width == 8 and len(shape) < 2):
            raise ValueError(f"tensor `{name}` has an invalid element width")
        if u64() != count * width // 8:
            raise ValueError(f"tensor `{name}` payload length mismatch")
        mass = u64()
        if len(shape) >= 2 and mass >= ROW_MASS_LIMIT:
            raise ValueError(f"tensor `{name}` max row mass violates the overflow bound")
        if name in seen:
            raise ValueError(f"deterministic artifact contains duplicate tensor `{name}`")
        seen.add(name)
        t = Tensor(name, shape, width=width)
        if width == 8:
            rows = count // shape[-1] if shape[-1] else 0
            if u64() != rows:
                raise ValueError(f"tensor `{name}` scale count mismatch")
            pad(name)
            t.q = np.frombuffer(take(count), dtype=np.int8).reshape(shape)
            pad(name)
            t.scale = np.frombuffer(take(rows * 4), dtype="<i4").astype(np.int32)
            v = t.values()
            if v.min(initial=0) < -2**31 or v.max(initial=0) > 2**31 - 1:
                raise ValueError(f"tensor `{name}` has q * scale values outside i32")
        else:
            pad(name)
            t.bits = np.frombuffer(take(count * width // 8), dtype="<i2" if width == 16 else "<i4").astype(np.int32)
            t.bits = t.bits.reshape(shape)
        if verify_mass and max_row_mass(shape, t.values()) != mass:
            raise ValueError(f"tensor `{name}` max row mass field does not match its values")
        out.append(t)
    if cur != len(data):
        raise ValueError("deterministic artifact has trailing bytes after tensor payloads")
    return out


_SAFETENSORS_DTYPES = {"F16": ("<f2", 2), "BF16": ("<u2", 2), "F32": ("<f4", 4), "F64": ("<f8", 8)}


def read_safetensors(data: bytes) -> dict[str, np.ndarray]:
    """float32 views of every tensor of a .safetensors file (F16 / BF16 / F32 /
    F64 sources, as the reference converter's decode_scalar reads them)."""
    n = struct.unpack("<Q", data[:8])[0]
    header = json.loads(data[8:8 + n])
    base = 8 + n
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        if info["dtype"] not in _SAFETENSORS_DTYPES:
            raise ValueError(f"unsupported tensor dtype {info['dtype']}")
        fmt, size = _SAFETENSORS_DTYPES[info["dtype"]]
        a, b = info["data_offsets"]
        raw = np.frombuffer(data[base + a:base + b], dtype=fmt)
        if info["dtype"] == "BF16":
            vals = (raw.astype(np.uint32) << 16).view(np.float32)
        else:
            vals = raw.astype(np.float32)
        out[name] = vals.reshape(info["shape"])
    return out


def convert_safetensors(data: bytes, int8: bool = False) -> bytes:
    """convert_model_to_det_num_wgt_artifact (converter main.rs:218-320):
    tensors in sorted name order, values through f32_to_wgt, the row-mass
    bound for rank >= 2 tensors, i16 storage when every value fits. With
    int8, writes detwgt-q8 and stores every exactly factoring matrix at width 8."""
    src = read_safetensors(data)
    tensors = [Tensor(name, tuple(src[name].shape), bits=f32_to_wgt(src[name])) for name in sorted(src)]
    return encode_q8(tensors) if int8 else encode_v2(tensors)


def main(argv: list[str]) -> int:
    if len(argv) >= 3 and argv[0] == "convert":
        data = open(argv[1], "rb").read()
        out = convert_safetensors(data, int8="--int8" in argv[3:])
        open(argv[2], "wb").write(out)
        print(f"wrote {argv[2]}: {len(out)} bytes")
        return 0
    if len(argv) == 2 and argv[0] == "audit":
        for t in parse(open(argv[1], "rb").read(), verify_mass=True):
            v = t.values()
            print(f"{t.name} shape={list(t.shape)} width={t.width} max_row_mass={max_row_mass(t.shape, v)}")
        return 0
    print("usage: python -m rasterdet.detwgt convert model.safetensors out.detwgt [--int8]\n"
          "       python -m rasterdet.detwgt audit artifact.detwgt")
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
