"""The allocation-free argmax entry point (det_argmax_first_noalloc) through
the C ABI: its index equals det_argmax_first's on consecutive calls, the
later ones with smaller inputs (the shared per-GPU scratch keeps the earlier
call's contents), and inputs past its fixed maximum are rejected."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
rd = pytest.importorskip("rasterdet")


@pytest.fixture(scope="module")
def ctx():
    c = rd.Context(0)
    yield c
    c.close()


def test_noalloc_argmax_equals_argmax_first_on_shrinking_inputs(ctx):
    out = ctx.empty(1, dtype=np.uint32)
    for n, seed, tie in [(1 << 24, 1, 12345678), (262144, 2, 70000), (1000, 3, 7), (1, 4, 0)]:
        rng = np.random.default_rng(seed)
        x = rng.integers(-1000, 1000, size=n).astype(np.int32)
        x[tie] = 5000
        if n > 1:
            x[n - 1] = 5000  # a later tie: the first index wins
        xd = ctx.to_device(x)
        ctx.argmax_first_noalloc(xd, n, out)
        got = int(out.numpy()[0])  # the copy back synchronizes the stream
        assert got == ctx.argmax_first(xd, n) == tie, n


def test_noalloc_argmax_rejects_sizes_past_its_maximum(ctx):
    out = ctx.empty(1, dtype=np.uint32)
    xd = ctx.to_device(np.zeros(4, dtype=np.int32))
    with pytest.raises(rd.DetError) as e:
        ctx.argmax_first_noalloc(xd, (1 << 24) + 1, out)  # rejected before any launch
    assert e.value.status == 1 and "at most 16777216" in str(e.value)
    with pytest.raises(rd.DetError) as e:
        ctx.argmax_first_noalloc(xd, 0, out)
    assert e.value.status == 2
