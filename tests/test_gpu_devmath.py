"""The product's integer arithmetic (det_arith.h) as the GPU executes it,
against the oracle: the device build of inv_sqrt_acc takes its own path (a
hardware reciprocal-square-root estimate refined by Newton steps, decided in
floating point away from the decision boundaries and by the exact integer
search near them), the division of the mean its own branch-free reciprocal
path, and both their own 64x64->128-bit products, which the host build of the
same header never compiles. The driver (tests/devmath/
gpu_devmath.hip) is built in-tree before the run. Its inputs include both
decision boundaries of inv_sqrt_acc (c^2 x = 2^64 and (2 c^2 + 2 c + 1) x =
2^65) and exact multiples and halves for the division. The device forms of
requant and mul_sat (32-bit halves around the rounding sum), the clamping
add_sat / sub_sat and add_sat64_nn are checked on their saturation edges and
exact ties as well."""
import pathlib
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = pathlib.Path(__file__).resolve().parent / "devmath" / "build" / "gpu_devmath"


def test_device_inv_sqrt_and_rms_scale_match_oracle():
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built (make -C tests/devmath)")
    res = subprocess.run([str(BIN), "2000000"], capture_output=True, text=True, timeout=100)
    rows = {}
    for line in res.stdout.splitlines():
        if line and not line.startswith(" "):
            name, n, bad = line.split()
            rows[name] = (int(n), int(bad))
    assert res.returncode == 0, res.stdout + res.stderr
    assert set(rows) == {"gpu_inv_sqrt_acc", "gpu_div_rte_nonneg_u32", "gpu_rms_scale", "gpu_requant", "gpu_mul_sat",
                         "gpu_add_sat", "gpu_sub_sat", "gpu_add_sat64_nn"}, res.stdout
    assert all(bad == 0 and n > 0 for n, bad in rows.values()), res.stdout
