"""CPU-side checks of the product library: it loads, exports every symbol the
C-ABI header declares, and its host-side pieces (synthetic GGUF generator,
GGUF/config parsing through backend construction errors) behave like the
reference.  No GPU compute is called here."""
import ctypes as C

import numpy as np
import pytest

import rust_interference_engine_amd as R
from rust_interference_engine_amd import synth


@pytest.fixture(scope="module")
def lib():
    return R.lib()


def test_library_exports_every_declared_symbol(lib):
    names = R._lib.declared_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n


@pytest.mark.parametrize("arch", ["llama", "qwen2", "qwen3", "phi3", "gemma", "gemma2", "gemma3", "granite", "qwen3moe", "qwen2moe"])
def test_synth_tiny_matches_oracle_bytes(oracle, arch):
    for ty in (0, 1, 30, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14):
        a = synth.build(synth.tiny(arch, ty))
        b = oracle.synth_build(oracle.synth_spec("tiny-" + arch, ty))
        assert a == b, (arch, ty)


def test_synth_preset_matches_oracle_bytes(oracle):
    for name, ty in (("smollm2-360m", 2), ("qwen3-0.6b", 12)):
        assert synth.build(synth.preset(name, ty)) == oracle.synth_build(oracle.synth_spec(name, ty))


def test_synth_presets_fall_back_like_llama_quantize(oracle):
    """testing.rs:202-210: k-quants need multiples of 256"""
    s = synth.preset("smollm2-360m", synth.Q4_K)
    assert s.wtype == synth.Q8_0 and s.embd_type == synth.Q8_0
    s = synth.preset("qwen3-1.7b", synth.Q4_0)
    assert s.embd_type == synth.Q6_K and s.tied_output == 1


def test_baseline_mode_statistics(oracle):
    """mode 1: N(0, 0.02) through quantize::q4_0; unit norms; RoPE base in the metadata;
    identical for any thread count."""
    import ggml_np as G
    from gguf_np import GGUF

    s = synth.baseline_llama31_8b_q4_0()
    s.n_layer, s.n_vocab, s.n_embd, s.n_ff, s.n_head, s.n_head_kv = 1, 1024, 512, 1024, 4, 2
    a = synth.build(s, n_threads=1)
    assert a == synth.build(s, n_threads=7)
    g = GGUF(a)
    assert abs(g.get("llama.rope.freq_base") - 5e5) < 1
    ty, dims, raw = g.tensors["blk.0.ffn_up.weight"]
    assert ty == synth.Q4_0
    w = G.dequantize(ty, raw, int(np.prod(dims)))
    assert abs(w.std() - 0.02) < 0.002 and abs(w.mean()) < 1e-3
    assert np.all(G.dequantize(0, g.tensors["blk.0.attn_norm.weight"][2], 512) == 1.0)
    assert g.tensors["output.weight"][0] == synth.Q4_0
    # the oracle parses the same image
    m = oracle.Model(a)
    assert m.cfg["n_layer"] == 1 and m.cfg["output_type"] == synth.Q4_0


def test_create_reports_reference_error_classes(lib):
    """Format / Unsupported errors cross the ABI as codes with messages (error.rs:5-29)."""
    err = C.create_string_buffer(512)
    code = C.c_int32(0)
    cfg = lib.rie_hip_default_config()
    junk = np.frombuffer(b"NOTAGGUF" + b"\0" * 64, np.uint8)
    h = lib.rie_hip_create(junk.ctypes.data, junk.size, C.byref(cfg), C.byref(code), err, 512)
    assert not h and code.value == -2 and b"bad magic" in err.value
    hdr = np.frombuffer(b"GGUF" + (7).to_bytes(4, "little") + b"\0" * 64, np.uint8)
    h = lib.rie_hip_create(hdr.ctypes.data, hdr.size, C.byref(cfg), C.byref(code), err, 512)
    assert not h and code.value == -3 and b"version 7" in err.value
    g = synth.build(synth.tiny("llama", synth.Q4_0))
    # unknown architecture: rewrite the metadata value 'llama' → 'llamb'
    bad = g.replace(b"\x05\x00\x00\x00\x00\x00\x00\x00llama", b"\x05\x00\x00\x00\x00\x00\x00\x00llamb", 1)
    arr = np.frombuffer(bad, np.uint8)
    h = lib.rie_hip_create(arr.ctypes.data, arr.size, C.byref(cfg), C.byref(code), err, 512)
    assert not h and code.value == -3 and b"architecture 'llamb'" in err.value


def test_kv_type_parse():
    assert R.KvType.parse("turbo4") == R.KvType.TURBO4 and R.KvType.parse("q8") == R.KvType.Q8_0
    assert R.KvType.parse("f16") == R.KvType.F16 and R.KvType.parse("x") is None


def test_argmax_first_max():
    assert R.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert R.argmax(np.array([np.nan, 1, 1], np.float32)) == 1
