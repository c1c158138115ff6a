"""CPU-side checks of the C ABI: the library loads, exports exactly what
include/rtgpu.h declares, and the host-side validation that runs before any
GPU work returns the reference's messages."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from rusttorch_amd import _lib, synth
from rusttorch_amd.gpt2 import Gpt2Config, Gpt2Error, Gpt2Model

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rtgpu.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rtg_[a-z_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (rtg_[a-z_]+)$", out, flags=re.M))
    assert set(names) <= exported
    assert lib.rtg_version().decode().startswith("rtgpu")


def test_missing_weight_error_before_gpu():
    sh = synth.SHAPES["tiny"]
    sd = synth.make_weights(sh)
    del sd["h.1.mlp.c_fc.bias"]
    with pytest.raises(Gpt2Error, match=r"^Missing weight: h\.1\.mlp\.c_fc\.bias$"):
        Gpt2Model.from_state_dict(sd, Gpt2Config(10, 16, 8, 2, 2))
    with pytest.raises(Gpt2Error, match=r"^Missing weight: wte\.weight$"):
        Gpt2Model.from_state_dict({}, Gpt2Config(10, 16, 8, 2, 2))


def test_shape_mismatch_error_before_gpu():
    sh = synth.SHAPES["tiny"]
    sd = synth.make_weights(sh)
    sd["h.0.attn.c_attn.weight"] = sd["h.0.attn.c_attn.weight"].T.copy()
    with pytest.raises(Gpt2Error, match=r"Shape mismatch for h\.0\.attn\.c_attn\.weight"):
        Gpt2Model.from_state_dict(sd, Gpt2Config(10, 16, 8, 2, 2))


def test_safetensors_errors(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(b"\x00" * 4)
    with pytest.raises(Gpt2Error, match="^Failed to load safetensors: Invalid safetensors format: File too small"):
        Gpt2Model.from_safetensors(str(p), Gpt2Config(10, 16, 8, 2, 2))
    with pytest.raises(Gpt2Error, match="^Failed to load safetensors: I/O error"):
        Gpt2Model.from_safetensors(str(tmp_path / "nope.safetensors"), Gpt2Config(10, 16, 8, 2, 2))
    # a well-formed file missing a tensor reaches the name check
    sh = synth.SHAPES["tiny"]
    sd = synth.make_weights(sh)
    del sd["ln_f.bias"]
    q = tmp_path / "partial.safetensors"
    synth.write_safetensors(str(q), sd)
    with pytest.raises(Gpt2Error, match=r"^Missing weight: ln_f\.bias$"):
        Gpt2Model.from_safetensors(str(q), Gpt2Config(10, 16, 8, 2, 2))


def test_no_device_fails_loudly():
    from tests.conftest import gpu_available
    if gpu_available():
        pytest.skip("a GPU is present")
    sh = synth.SHAPES["tiny"]
    with pytest.raises(Gpt2Error, match="rtgpu requires an MI355X|no HIP device"):
        Gpt2Model.from_state_dict(synth.make_weights(sh), Gpt2Config(10, 16, 8, 2, 2))


def test_synth_matches_numpy_spec():
    sh = synth.SHAPES["mini"]
    a = synth.make_weights(sh)
    b = synth.make_weights(sh, use_numpy=True)
    for k in a:
        assert np.array_equal(a[k], b[k]), k


def test_bf16_rounding():
    x = np.array([1.0, -2.0, 1.00390625, 1.0078125, 3.0e38, np.inf], np.float32)
    bits = synth.f32_to_bf16_bits(x)
    assert bits[0] == 0x3F80 and bits[1] == 0xC000  # safetensors.rs:755-775 values
    assert synth.bf16_bits_to_f32(bits)[2] == 1.0  # tie rounds to even
    assert synth.bf16_bits_to_f32(bits)[3] == 1.0078125
    assert np.isinf(synth.bf16_bits_to_f32(bits)[5])
