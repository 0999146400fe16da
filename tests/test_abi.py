"""CPU-side checks of the boundary: the C-ABI library loads, exports every symbol that
include/llmembed.h declares, and fails cleanly (no crash, a clear error) without a GPU; the
GGUF writer/reader round-trips and matches the reference reader's rules."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import llmembed
from llmembed import _lib, gguf, quant, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "llmembed.h")


def declared_symbols():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(lle_[a-z0-9_]+)\s*\(", src)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (lle_\w+)", out))
    assert set(declared_symbols()) <= exported


def test_no_cpu_fallback_without_device():
    """In a container without a GPU the product fails loudly (EDEVICE), never computes on CPU."""
    if os.path.exists("/dev/kfd") and os.environ.get("HIP_VISIBLE_DEVICES", "") != "-1":
        pytest.skip("a GPU device node is present")
    lib = _lib.lib()
    assert lib.lle_abi_version() == 1
    rc = lib.lle_init(0)
    assert rc == -2 and b"device" in lib.lle_last_error()
    h = C.c_void_p()
    assert lib.lle_model_load_gguf(b"/nonexistent.gguf", C.byref(h)) != 0
    out = np.zeros(32, np.float32)
    blk = np.zeros(34, np.uint8)
    assert lib.lle_dequant(8, blk.ctypes.data, 32, out.ctypes.data) == -2


def test_gguf_roundtrip(tmp_path):
    rng = np.random.default_rng(0)
    w = rng.standard_normal((4, 256)).astype(np.float32)
    q = quant.quantize(quant.Q6_K, w, rng).reshape(-1)
    p = str(tmp_path / "t.gguf")
    gguf.write(p, [("a.u32", gguf.T_U32, 7), ("a.f32", gguf.T_F32, 1.5), ("a.s", gguf.T_STR, "x"),
                   ("a.arr", gguf.T_ARR, (gguf.T_STR, ["p", "q"]))],
               [("w", [256, 4], quant.Q6_K, q), ("v", [3], quant.F32, np.arange(3, dtype=np.float32).view(np.uint8))])
    g = gguf.read(p)
    assert g.get_u32("a.u32") == 7 and g.get_f32("a.f32") == 1.5 and g.get_str("a.s") == "x"
    assert g.get_u32("a.f32") is None  # strict type switch (reader.go:293-332)
    assert g.data_offset % 32 == 0
    assert np.array_equal(np.asarray(g.tensor_bytes("w")), q)
    assert g.tensors["w"].byte_size == 4 * 210
    assert np.array_equal(np.asarray(g.tensor_bytes("v")).view(np.float32), np.arange(3, dtype=np.float32))


def test_gguf_rejects_bad_magic_and_version(tmp_path):
    p = str(tmp_path / "bad.gguf")
    open(p, "wb").write(b"GGUX" + b"\0" * 20)
    with pytest.raises(gguf.GGUFError, match="invalid magic"):
        gguf.read(p)
    open(p, "wb").write(b"GGUF" + (4).to_bytes(4, "little") + b"\0" * 16)
    with pytest.raises(gguf.GGUFError, match="unsupported version"):
        gguf.read(p)


def test_synthetic_model_is_deterministic_and_complete(small_spec):
    p = synth.model_path(small_spec, "Q4_K_M", 100)
    g = gguf.read(p)
    assert g.get_u32("nomic-bert.block_count") == 2
    assert g.get_f32("nomic-bert.rope.freq_base") == 1000.0
    names = {"token_embd.weight", "token_types.weight", "token_embd_norm.weight", "token_embd_norm.bias"}
    for l in range(2):
        for s in ("attn_qkv.weight", "attn_output.weight", "attn_output_norm.weight", "attn_output_norm.bias",
                  "ffn_up.weight", "ffn_gate.weight", "ffn_down.weight", "layer_output_norm.weight",
                  "layer_output_norm.bias"):
            names.add(f"blk.{l}.{s}")
    assert names <= set(g.tensors)
    assert g.tensors["blk.0.attn_qkv.weight"].type == quant.Q5_K
    assert g.tensors["blk.0.ffn_down.weight"].type == quant.Q6_K
    assert g.tensors["blk.1.ffn_down.weight"].type == quant.Q4_K
    kvs, tensors = synth.build_tensors(small_spec, "Q4_K_M", 100)
    assert np.array_equal(np.asarray(g.tensor_bytes("blk.1.ffn_up.weight")),
                          [t for t in tensors if t[0] == "blk.1.ffn_up.weight"][0][3])
