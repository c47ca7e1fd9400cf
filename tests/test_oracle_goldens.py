"""The oracle's certificate: every det_* commitment the reference pinned in
testdata/det_commitment_goldens.json (src/runtime/det_goldens.rs) must be
reproduced bit-exactly by the CPU restatement."""
import pytest

import fixtures
import oracle_lib


@pytest.mark.parametrize("name", ["donor_ple", "no_donor_ple"])
def test_oracle_reproduces_reference_det_goldens(name):
    cfg, wgt, prompt, steps = fixtures.golden_fixture(name)
    model = oracle_lib.OracleModel(cfg).load_detwgt(wgt).finalize()
    got = model.capture(prompt, steps)
    exp = fixtures.golden_expected(name)
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    for i, (g, e) in enumerate(zip(got["decode_steps"], exp["decode_steps"])):
        assert g == e, f"decode step {i}"
    assert len(got["decode_steps"]) == len(exp["decode_steps"])
    assert got["end_to_end"] == exp["end_to_end"]


@pytest.mark.parametrize("name", ["donor_ple", "no_donor_ple"])
def test_i32_storage_gives_identical_commitments(name):
    # detwgt v2 invariant: storage width is representation only
    # (DETWGT_V2_FORMAT.md; schedule_parity.rs:98-139).
    cfg, _, prompt, _ = fixtures.golden_fixture(name)
    wide = fixtures.encode_detwgt(fixtures.golden_tensors(), force_i32=True)
    model = oracle_lib.OracleModel(cfg).load_detwgt(wide).finalize()
    got = model.capture(prompt, 8)
    exp = fixtures.golden_expected(name)
    assert got["prefill"] == exp["prefill"]
    assert got["decode_steps"] == exp["decode_steps"][:8]


@pytest.mark.parametrize("threads", [1, 2, 3, 8])
def test_thread_count_invariance(threads):
    # schedule_parity.rs:55-83: committed bytes are identical for every pool size.
    cfg, wgt, prompt, _ = fixtures.golden_fixture("no_donor_ple")
    oracle_lib.set_threads(threads)
    try:
        got = oracle_lib.OracleModel(cfg).load_detwgt(wgt).finalize().capture(prompt, 4)
    finally:
        oracle_lib.set_threads(1)
    exp = fixtures.golden_expected("no_donor_ple")
    assert got["prefill"] == exp["prefill"]
    assert got["decode_steps"] == exp["decode_steps"][:4]


@pytest.mark.parametrize("group,threads", [(2, 1), (5, 3), (16, 8)])
def test_slab_group_invariance(group, threads):
    # token rows grouped per slab work item (each weight row read once per
    # group) give the reference schedule's commitments: every output element
    # adds its terms in column order either way
    cfg, wgt, prompt, _ = fixtures.golden_fixture("donor_ple")
    oracle_lib.set_threads(threads)
    oracle_lib.set_slab_group(group)
    try:
        got = oracle_lib.OracleModel(cfg).load_detwgt(wgt).finalize().capture(prompt, 4)
    finally:
        oracle_lib.set_threads(1)
        oracle_lib.set_slab_group(1)
    exp = fixtures.golden_expected("donor_ple")
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"][:4]


@pytest.mark.parametrize("width", [16, 32])
def test_slab_group_matches_per_token_gemv(width):
    # the grouped slab against one GEMV per token row, ragged token counts
    # and row lengths, values at the ends of the storage range
    import numpy as np
    rng = np.random.default_rng(width)
    info = np.iinfo(np.int16 if width == 16 else np.int32)
    for m, n, k in [(1, 7, 5), (17, 33, 129), (40, 64, 1000)]:
        w = rng.integers(info.min, info.max, size=(n, k), endpoint=True).astype(info.dtype)
        a = rng.integers(-(1 << 31), 1 << 31, size=(m, k)).astype(np.int32)
        exp = np.stack([oracle_lib.det_linear(w, a[t]) for t in range(m)])
        for group, threads in [(3, 1), (16, 4)]:
            oracle_lib.set_slab_group(group)
            try:
                got = oracle_lib.det_linear_slab(w, a, threads=threads)
            finally:
                oracle_lib.set_slab_group(1)
            assert np.array_equal(got, exp), (m, n, k, group)


def test_loader_fails_closed():
    cfg, wgt, _, _ = fixtures.golden_fixture("no_donor_ple")
    bad_version = wgt[:8] + (1).to_bytes(4, "little") + wgt[12:]
    with pytest.raises(oracle_lib.OracleError):
        oracle_lib.OracleModel(cfg).load_detwgt(bad_version)
    with pytest.raises(oracle_lib.OracleError):
        oracle_lib.OracleModel(cfg).load_detwgt(wgt + b"\0")  # trailing bytes
    with pytest.raises(oracle_lib.OracleError):
        oracle_lib.OracleModel(cfg).load_detwgt(wgt[:-2])  # truncated


def test_loader_rejects_wrapping_and_oversized_headers():
    # element count x width overflows u64 (2^62 x 4 = 2^64 wraps to 0): the
    # reference's checked_mul rejects it (gemma/io.rs:327-331); a rank larger
    # than the remaining bytes ends the artifact before any allocation
    import struct
    cfg, _, _, _ = fixtures.golden_fixture("no_donor_ple")
    head = b"DNWGTV0\0" + struct.pack("<IIQ", 2, 1, 1)
    rec = struct.pack("<I", 1) + b"w" + struct.pack("<I", 2) + struct.pack("<QQ", 1 << 31, 1 << 31)
    rec += struct.pack("<QIQQ", 1 << 62, 32, 0, 0)
    with pytest.raises(oracle_lib.OracleError, match="payload byte count overflowed") as e:
        oracle_lib.OracleModel(cfg).load_detwgt(head + rec)
    assert e.value.status == 1
    with pytest.raises(oracle_lib.OracleError, match="ended unexpectedly"):
        oracle_lib.OracleModel(cfg).load_detwgt(head + struct.pack("<I", 1) + b"w" + struct.pack("<I", 0xFFFFFFFF))
