"""CPU cross-check of the product's integer arithmetic (det_arith.h, the
header the HIP kernels compile) against the oracle, on random and edge-case
inputs. Runs without a GPU: the header is built for the host by hipcc."""
import pathlib
import shutil
import subprocess

import pytest

import oracle_lib

HERE = pathlib.Path(__file__).resolve().parent / "devmath"


@pytest.mark.skipif(shutil.which("/opt/rocm/bin/hipcc") is None and shutil.which("hipcc") is None,
                    reason="hipcc not available")
def test_device_arithmetic_matches_oracle():
    oracle_lib.build_oracle()
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    res = subprocess.run([str(HERE / "build" / "fuzz_devmath"), "100000"], capture_output=True, text=True)
    rows = [line.split() for line in res.stdout.splitlines() if line and not line.startswith(" ")]
    assert rows, res.stdout + res.stderr
    bad = {name: (int(n), int(b)) for name, n, b in rows if int(b)}
    assert res.returncode == 0 and not bad, res.stdout
    names = {r[0] for r in rows}
    assert {"requant", "add_sat64_nn", "inv_sqrt_acc", "inv_sqrt_acc_edges", "softmax_exp_all_gaps", "softmax_weight",
            "softmax_weight_recip", "div_rte_nonneg", "sin_cos", "rope", "gelu"} <= names
