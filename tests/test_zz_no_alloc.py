"""lle_embed_packed_noalloc (no device allocation: activations in a fixed per-device array)
against lle_embed_packed_async, the entry point it is a variant of: the same rows bit for bit,
on two calls in a row whose second input is smaller, and through every GEMM schedule the token
counts select. Batches that do not fit the array are rejected before any launch."""
import ctypes as C

import numpy as np
import pytest

from llmembed import Embedder, _hip, synth
from llmembed._lib import check, lib

pytestmark = pytest.mark.gpu

SCRATCH = 32 * 1024 * 1024


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def emb(gpu, small_spec):
    return Embedder.load(synth.model_path(small_spec, "Q8_0", 100))


def packed(rng, vocab, lens):
    seqs = [rng.integers(0, vocab, n).astype(np.int32) for n in lens]
    return np.concatenate(seqs), np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)


def run(entry, m, ids, off, L, D, stream):
    B, T = off.size - 1, int(ids.size)
    di, do_ = _hip.DeviceBuffer.from_array(ids), _hip.DeviceBuffer.from_array(off)
    dy = _hip.DeviceBuffer(B * D * 4)
    check(entry(m.h, di.ptr, do_.ptr, B, T, L, D, dy.ptr, stream.h))
    stream.synchronize()
    return dy.download((B, D), np.float32)


@pytest.mark.parametrize("lens", [
    ([100, 3, 64, 1, 77], [8]),          # 245 rows (split-K GEMMs), then 8 (fused small schedule)
    ([512], [40, 2, 17]),                # the 512-token maximum in one sequence, then 59 rows
    ([16, 16, 16, 16], [1]),             # 64 rows, then a single token
])
def test_noalloc_matches_packed_async(emb, lens):
    m = emb.model()
    D = emb.dim()
    rng = np.random.default_rng(sum(lens[0]))
    stream = _hip.Stream()
    for call, ln in enumerate(lens):
        ids, off = packed(rng, m.vocab_size, ln)
        L = max(ln)
        print(f"noalloc call {call}: lens={ln} T={ids.size} L={L}", flush=True)
        ref = run(lib().lle_embed_packed_async, m, ids, off, L, D, stream)
        got = run(lib().lle_embed_packed_noalloc, m, ids, off, L, D, stream)
        assert np.array_equal(bits(got), bits(ref)), (call, ln)
        assert np.abs(np.linalg.norm(got.astype(np.float64), axis=1) - 1.0).max() < 1e-5
    st = C.c_int32(-1)
    check(lib().lle_model_status(m.h, C.byref(st)))
    assert st.value == 0


def test_noalloc_rows_equal_single_embeds(emb):
    """Each row also equals lle_embed of that sequence (the host entry's own workspace)."""
    m = emb.model()
    D = emb.dim()
    rng = np.random.default_rng(9)
    lens = [30, 5, 200]
    ids, off = packed(rng, m.vocab_size, lens)
    got = run(lib().lle_embed_packed_noalloc, m, ids, off, max(lens), D, _hip.Stream())
    for b, n in enumerate(lens):
        assert np.array_equal(bits(got[b]), bits(emb.embed(ids[off[b]:off[b + 1]]))), n


def test_noalloc_rejects_batches_past_the_array(emb):
    """Rejected on the host with LLE_EINVAL and the bytes needed; nothing is launched."""
    m = emb.model()
    D = emb.dim()
    for lens in ([1000], [64] * 40):  # 1000 tokens: 37 MB; 40 x 64 tokens (no split-K): 43 MB
        ids = np.zeros(sum(lens), np.int32)
        off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        di, do_ = _hip.DeviceBuffer.from_array(ids), _hip.DeviceBuffer.from_array(off)
        dy = _hip.DeviceBuffer(len(lens) * D * 4)
        rc = lib().lle_embed_packed_noalloc(m.h, di.ptr, do_.ptr, len(lens), int(ids.size), max(lens), D, dy.ptr, None)
        msg = lib().lle_last_error().decode()
        assert rc == -1 and "bytes of scratch" in msg and str(SCRATCH) in msg, (lens, rc, msg)
