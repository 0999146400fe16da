"""CPU tests of the native GGUF loader's failure paths (lle_model_load_gguf).

Every malformed file must be rejected with the right LLE_E* code and message before the device
is touched, so these run without a GPU. Cases follow the reference reader and loader:
internal/gguf/reader.go:219-280 (magic, version, truncated header / KV pairs / tensor table) and
internal/embed/bert.go:98-139 (metadata keys, `tensor %q not found`, the mmap slice of a tensor's
data), plus what the reference leaves to Go's runtime (overflowing dims, nested arrays, data past
the end of the file), which the C loader must turn into errors.
"""
import ctypes as C
import struct

import pytest

from llmembed import _lib

EINVAL, EUNSUPPORTED, EIO, ENOTFOUND = -1, -4, -5, -6
MAGIC = 0x46554747
U32, F32, STR, ARR = 4, 6, 8, 9


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, t, v):
    out = _str(key) + struct.pack("<I", t)
    if t == U32:
        return out + struct.pack("<I", v)
    if t == F32:
        return out + struct.pack("<f", v)
    if t == STR:
        return out + _str(v)
    raise ValueError(t)


def _tinfo(name, dims, ty, off):
    return _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", ty, off)


META = [("nomic-bert.block_count", U32, 2), ("nomic-bert.embedding_length", U32, 768),
        ("nomic-bert.feed_forward_length", U32, 3072), ("nomic-bert.attention.head_count", U32, 12),
        ("nomic-bert.context_length", U32, 2048), ("nomic-bert.attention.layer_norm_epsilon", F32, 1e-12),
        ("nomic-bert.rope.freq_base", F32, 1000.0)]


def tensor_names(n_layer=2):
    names = ["token_embd.weight", "token_types.weight", "token_embd_norm.weight", "token_embd_norm.bias"]
    for l in range(n_layer):
        names += [f"blk.{l}.{s}" for s in (
            "attn_qkv.weight", "attn_output.weight", "ffn_up.weight", "ffn_gate.weight", "ffn_down.weight",
            "attn_output_norm.weight", "attn_output_norm.bias", "layer_output_norm.weight",
            "layer_output_norm.bias")]
    return names


def gguf_bytes(kvs=META, tensors=None, version=3, data=b""):
    """tensors: [(name, dims, type, offset)]; default: every tensor an F32 [4] at its own offset."""
    if tensors is None:
        tensors = [(n, [4], 0, 32 * i) for i, n in enumerate(tensor_names())]
        data = b"\0" * (32 * len(tensors))
    head = struct.pack("<IIQQ", MAGIC, version, len(tensors), len(kvs))
    head += b"".join(_kv(*kv) for kv in kvs)
    head += b"".join(_tinfo(*t) for t in tensors)
    head += b"\0" * (((len(head) + 31) & ~31) - len(head))
    return head + data


def load(tmp_path, blob, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(blob)
    lib = _lib.lib()
    h = C.c_void_p()
    rc = lib.lle_model_load_gguf(str(p).encode(), C.byref(h))
    assert not h.value  # nothing is handed out on failure
    return rc, lib.lle_last_error().decode()


def test_bad_magic(tmp_path):
    rc, msg = load(tmp_path, b"GGUX" + gguf_bytes()[4:])
    assert rc == EIO and "invalid magic: 0x58554747 (expected 0x46554747)" in msg


@pytest.mark.parametrize("version", [1, 4, 0xFFFFFFFF])
def test_bad_version(tmp_path, version):
    rc, msg = load(tmp_path, gguf_bytes(version=version))
    assert rc == EIO and f"unsupported version: {version}" in msg


def test_version_2_accepted_by_the_parser(tmp_path):
    """Version 2 parses like 3 (reader.go:233); the all-F32 [4] tensors then fail shape validation."""
    rc, msg = load(tmp_path, gguf_bytes(version=2))
    assert rc == EINVAL and "token_embd.weight: shape [4, 1]" in msg


@pytest.mark.parametrize("cut", [0, 3, 4, 7, 8, 23])
def test_truncated_header(tmp_path, cut):
    rc, msg = load(tmp_path, gguf_bytes()[:cut])
    assert rc == EIO
    if cut < 4:  # a short read leaves the magic 0 (reader.go:228-231)
        assert "invalid magic: 0x00000000" in msg
    elif cut < 8:
        assert "unsupported version: 0" in msg
    else:
        assert msg == "gguf: reading header: truncated"


def test_truncated_kv_section(tmp_path):
    full = gguf_bytes()
    kv_start = 24
    kv_len = sum(len(_kv(*kv)) for kv in META)
    for cut in (kv_start + 5, kv_start + kv_len // 2, kv_start + kv_len - 1):
        rc, msg = load(tmp_path, full[:cut])
        assert rc == EIO and "reading KV pair" in msg, (cut, msg)


def test_truncated_tensor_table(tmp_path):
    full = gguf_bytes()
    table = 24 + sum(len(_kv(*kv)) for kv in META)
    rc, msg = load(tmp_path, full[:table + 30])
    assert rc == EIO and "reading tensor 0" in msg
    n_before = len(_tinfo("token_embd.weight", [4], 0, 0)) + len(_tinfo("token_types.weight", [4], 0, 32))
    rc, msg = load(tmp_path, full[:table + n_before + 9])
    assert rc == EIO and "reading tensor 2" in msg


def test_string_length_past_end(tmp_path):
    blob = struct.pack("<IIQQ", MAGIC, 3, 0, 1) + struct.pack("<Q", 1 << 62) + b"key"
    rc, msg = load(tmp_path, blob)
    assert rc == EIO and "reading KV pair 0" in msg


def test_deeply_nested_array_rejected(tmp_path):
    """Arrays of arrays recurse in readValue; 10,000 levels in 120 KB must not exhaust the stack."""
    depth = 10000
    val = b"".join(struct.pack("<IQ", ARR, 1) for _ in range(depth)) + struct.pack("<IQ", U32, 0)
    blob = struct.pack("<IIQQ", MAGIC, 3, 0, 1) + _str("deep") + struct.pack("<I", ARR) + val
    rc, msg = load(tmp_path, blob)
    assert rc == EIO and "reading KV pair 0" in msg


def test_unknown_value_type(tmp_path):
    blob = struct.pack("<IIQQ", MAGIC, 3, 0, 1) + _str("k") + struct.pack("<I", 13) + b"\0" * 8
    rc, msg = load(tmp_path, blob)
    assert rc == EIO and "reading KV pair 0" in msg


def test_missing_metadata(tmp_path):
    rc, msg = load(tmp_path, gguf_bytes(kvs=META[2:]))
    assert rc == EINVAL and msg == "embed: missing model params in GGUF metadata"


def test_wrong_metadata_type_is_missing(tmp_path):
    """Getters type-switch strictly (reader.go:293-332): block_count stored as f32 reads as absent."""
    kvs = [("nomic-bert.block_count", F32, 2.0)] + META[1:]
    rc, msg = load(tmp_path, gguf_bytes(kvs=kvs))
    assert rc == EINVAL and "missing model params" in msg


def test_missing_tensor_first(tmp_path):
    rc, msg = load(tmp_path, gguf_bytes(tensors=[], data=b""))
    assert rc == ENOTFOUND and msg == 'tensor "token_embd.weight" not found'


def test_missing_tensor_later_layer(tmp_path):
    names = [n for n in tensor_names() if n != "blk.1.ffn_down.weight"]
    tensors = [(n, [4], 0, 32 * i) for i, n in enumerate(names)]
    rc, msg = load(tmp_path, gguf_bytes(tensors=tensors, data=b"\0" * (32 * len(tensors))))
    assert rc == ENOTFOUND and msg == 'tensor "blk.1.ffn_down.weight" not found'


def test_tensor_data_past_end_of_file(tmp_path):
    names = tensor_names()
    tensors = [(n, [4], 0, 32 * i) for i, n in enumerate(names)]
    tensors[5] = (names[5], [4], 0, 1 << 20)  # blk.0.attn_output.weight, 1 MiB past the data
    rc, msg = load(tmp_path, gguf_bytes(tensors=tensors, data=b"\0" * (32 * len(tensors))))
    assert rc == EIO and "blk.0.attn_output.weight: data past end of file" in msg


def test_tensor_data_cut_short(tmp_path):
    """The last tensor's bytes run past a truncated data section."""
    blob = gguf_bytes()
    rc, msg = load(tmp_path, blob[:-20])
    assert rc == EIO and "blk.1.layer_output_norm.bias: data past end of file" in msg


def test_offset_overflow(tmp_path):
    names = tensor_names()
    tensors = [(n, [4], 0, 32 * i) for i, n in enumerate(names)]
    tensors[0] = (names[0], [4], 0, (1 << 64) - 16)  # data_off + offset wraps
    rc, msg = load(tmp_path, gguf_bytes(tensors=tensors, data=b"\0" * (32 * len(tensors))))
    assert rc == EIO and "token_embd.weight: data past end of file" in msg


def test_element_count_overflow(tmp_path):
    """dims whose product wraps 2^64 (here to 0 bytes) must not pass the bounds check."""
    names = tensor_names()
    tensors = [(n, [4], 0, 32 * i) for i, n in enumerate(names)]
    tensors[0] = (names[0], [1 << 32, 1 << 32], 8, 0)
    rc, msg = load(tmp_path, gguf_bytes(tensors=tensors, data=b"\0" * (32 * len(tensors))))
    assert rc == EIO and "token_embd.weight: element count overflows" in msg


def test_byte_size_overflow(tmp_path):
    names = tensor_names()
    tensors = [(n, [4], 0, 32 * i) for i, n in enumerate(names)]
    tensors[0] = (names[0], [1 << 62], 0, 0)  # F32: 4 bytes each
    rc, msg = load(tmp_path, gguf_bytes(tensors=tensors, data=b"\0" * (32 * len(tensors))))
    assert rc == EIO and "token_embd.weight: byte size overflows" in msg


def test_dimension_above_int32(tmp_path):
    names = tensor_names()
    tensors = [(n, [4], 0, 32 * i) for i, n in enumerate(names)]
    tensors[0] = (names[0], [768, 1 << 31], 24, 0)  # I8 (1 byte each): fits the file check only if huge
    rc, msg = load(tmp_path, gguf_bytes(tensors=tensors, data=b"\0" * (32 * len(tensors))))
    assert rc == EIO and ("data past end of file" in msg or "above 2^31" in msg)


def test_shape_mismatch_rejected_before_device(tmp_path):
    rc, msg = load(tmp_path, gguf_bytes())
    assert rc == EINVAL and msg == "token_embd.weight: shape [4, 1], expected [768, -1]"


def test_head_dim_must_be_64(tmp_path):
    kvs = [kv if kv[0] != "nomic-bert.attention.head_count" else (kv[0], U32, 16) for kv in META]
    rc, msg = load(tmp_path, gguf_bytes(kvs=kvs))
    assert rc == EUNSUPPORTED and "head_dim must be 64" in msg


def test_implausible_block_count(tmp_path):
    kvs = [kv if kv[0] != "nomic-bert.block_count" else (kv[0], U32, 0x80000000) for kv in META]
    rc, msg = load(tmp_path, gguf_bytes(kvs=kvs))
    assert rc == EINVAL and "implausible block_count" in msg


def test_nonexistent_path(tmp_path):
    lib = _lib.lib()
    h = C.c_void_p()
    rc = lib.lle_model_load_gguf(str(tmp_path / "none.gguf").encode(), C.byref(h))
    assert rc == EIO and "No such file" in lib.lle_last_error().decode()
