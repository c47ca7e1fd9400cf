"""CPU checks of the boundary: the C-ABI library loads and exports every
entry point that include/detgpu.h declares (no compute calls)."""
import ctypes
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "detgpu.h"
LIB = ROOT / "raster-inference_amd" / "build" / "libdetgpu.so"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(det_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ["det_ctx_create", "det_matrix_upload", "det_linear", "det_linear_slab", "det_rms_norm",
                     "det_rope", "det_attention_causal", "det_model_load_detwgt", "det_session_prefill",
                     "det_session_decode", "det_capture", "det_layer_prefill", "det_layer_decode",
                     "det_decode_ple_input", "det_prefill_ple_inputs", "det_hidden_to_logits", "det_embed_tokens",
                     "det_kv_create", "det_kv_read_logical", "det_kv_commitment", "det_scratch_create"]:
        assert required in names


@pytest.mark.skipif(not LIB.exists(), reason="libdetgpu.so not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    lib.det_version.restype = ctypes.c_char_p
    assert b"gfx950" in lib.det_version()


def test_python_wrapper_binds_the_header():
    import rasterdet

    src = (ROOT / "raster-inference_amd" / "rasterdet" / "__init__.py").read_text()
    for n in declared_functions():
        assert f'"{n}"' in src, n
    assert rasterdet.TextConfig.from_json({"text_config": {
        "enable_moe_block": False, "hidden_activation": "gelu_pytorch_tanh", "head_dim": 2, "hidden_size": 4,
        "layer_types": ["sliding_attention"], "num_attention_heads": 1, "num_hidden_layers": 1,
        "num_key_value_heads": 1, "rms_norm_eps": 1e-6, "sliding_window": 4, "vocab_size": 9}}).hidden_size == 4


@pytest.mark.skipif(not LIB.exists(), reason="libdetgpu.so not built")
def test_native_synthetic_generator_matches_python_definition():
    import rasterdet
    from rasterdet import synthetic

    for seed, rows, cols, smax in [(1, 7, 13, 16), (12345, 33, 100, 256), (2**63 + 5, 3, 1, 1)]:
        q, s = rasterdet.synthetic_int8(seed, rows, cols, smax)
        q2, s2 = synthetic.fast_int8_matrix(seed, rows, cols, smax)
        assert (q == q2).all() and (s == s2).all()
        assert q.min() >= -127 and q.max() <= 127 and s.min() >= 1 and s.max() <= smax


@pytest.mark.skipif(not LIB.exists(), reason="libdetgpu.so not built")
@pytest.mark.parametrize("rows,cols,lim", [(1, 1, 5), (23, 17, 4096), (77, 300, 32767), (4, 3, 1)])
def test_native_i16_generator_equals_numpy(rows, cols, lim):
    # host-only: det_synthetic_i16 reproduces synthetic.fast_i16_matrix
    import rasterdet
    from rasterdet import synthetic
    seed = rows * 1000 + cols
    assert (rasterdet.synthetic_i16(seed, rows, cols, lim) == synthetic.fast_i16_matrix(seed, rows, cols, lim)).all()
