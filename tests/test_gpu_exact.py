"""LLE_PRECISION_F32: the reference CPU path's own f32 arithmetic on the GPU (GemmPrePacked32's
128-wide K chunks with FMA chains and unfused edge rows, internal/ggml/gemm_avx512.go:67-147;
sequential LayerNorm sums, DotF32 order and f64 exp, internal/ggml/ops_simd.go; MeanPool /
L2Normalize, internal/embed/pool.go). Embeddings and hidden states must equal the C oracle's
(the restatement of that path) bit for bit. (The softmax's exp is evaluated in float64 by the
GPU's exp and by glibc's; a last-ulp difference between the two would show here as a mismatch.
None occurs on these inputs.)"""
import ctypes as C

import numpy as np
import pytest

import oracle
from llmembed import Embedder, _hip, synth
from llmembed._lib import lib

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


_models = {}


def models(spec, mix, seed=100):
    key = (spec, mix, seed)
    if key not in _models:
        p = synth.model_path(spec, mix, seed)
        e = Embedder.load(p)
        e.model().set_precision("f32")
        _models[key] = (e, oracle.OracleModel(p))
    return _models[key]


def check_exact(got, ref, what):
    got, ref = np.atleast_2d(got), np.atleast_2d(ref)
    same = np.all(bits(got) == bits(ref), axis=1)
    mx = float(np.abs(got.astype(np.float64) - ref).max())
    print(f"{what}: {int(same.sum())}/{same.size} rows bit-equal, max abs {mx:.3e}", flush=True)
    assert same.all(), (what, mx)


@pytest.mark.parametrize("mix", ["Q8_0", "Q4_K_M", "Q6_K", "Q5_K", "F32"])
def test_exact_embed_equals_oracle(gpu, small_spec, mix):
    """Lengths 1..13 straddle the 6-row tiles (unfused edge rows), 64 and 130 span K-tile and
    GEMM-tile boundaries."""
    e, o = models(small_spec, mix)
    rng = np.random.default_rng(5)
    for L in (1, 5, 6, 7, 8, 13, 64, 130):
        ids = rng.integers(0, small_spec.vocab, L).astype(np.int32)
        check_exact(e.embed(ids), o.embed(ids), f"exact {mix} L={L}")


def test_exact_hidden_states_equal_oracle(gpu, small_spec):
    e, o = models(small_spec, "Q8_0")
    rng = np.random.default_rng(6)
    ids = rng.integers(0, small_spec.vocab, 23).astype(np.int32)
    mask = np.ones(23, np.int32)
    mask[[2, 9]] = 0  # interior masked keys: -1e9 scores, rows kept out of no pool here
    check_exact(e.model().forward(ids, mask), o.forward(ids, mask), "exact hidden L=23")


def test_exact_batch_equals_oracle_and_embed(gpu, small_spec):
    """EmbedBatch (packed rows: each sequence at its own length, as the reference embeds each
    text) equals the oracle's EmbedBatch and each row's Embed, bit for bit; Matryoshka too."""
    e, o = models(small_spec, "Q4_K_M")
    rng = np.random.default_rng(7)
    lens = [3, 17, 64, 1, 40, 12]
    B, L = len(lens), max(lens)
    ids = rng.integers(0, small_spec.vocab, (B, L)).astype(np.int32)
    mask = (np.arange(L)[None, :] < np.array(lens)[:, None]).astype(np.int32)
    mask[1, 5] = 0  # an interior zero
    batch = e.embed_padded(ids, mask)
    check_exact(batch, o.embed_batch(ids, mask), "exact batch")
    for b, n in enumerate(lens):
        assert np.array_equal(bits(e.embed(ids[b, :n], mask[b, :n])), bits(batch[b])), b
    e.set_target_dim(256)
    try:
        check_exact(e.embed_padded(ids, mask), o.embed_batch(ids, mask, out_dim=256), "exact matryoshka 256")
    finally:
        e.set_target_dim(768)


def test_exact_packed_device_entry(gpu, small_spec):
    e, o = models(small_spec, "Q8_0")
    m = e.model()
    D = small_spec.d_model
    rng = np.random.default_rng(8)
    lens = [9, 30, 2]
    seqs = [rng.integers(0, small_spec.vocab, n).astype(np.int32) for n in lens]
    packed = np.concatenate(seqs)
    off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    di, do_, dy = _hip.DeviceBuffer.from_array(packed), _hip.DeviceBuffer.from_array(off), _hip.DeviceBuffer(3 * D * 4)
    assert lib().lle_embed_packed_async(m.h, di.ptr, do_.ptr, 3, int(packed.size), max(lens), D, dy.ptr, None) == 0
    _hip.synchronize()
    got = dy.download((3, D), np.float32)
    check_exact(got, np.stack([o.embed(s) for s in seqs]), "exact packed device entry")


def test_exact_full_model_config1(gpu, full_spec):
    """Config 1 on the full 12-layer Q8_0 model."""
    e, o = models(full_spec, "Q8_0", synth.CONFIG_SEED + 1)
    ids, _ = synth.config_inputs(1)
    check_exact(e.embed(ids[0]), o.embed(ids[0]), "exact c1")


def test_exact_full_model_config3_rows(gpu, full_spec):
    """Config 3's model (Q4_K_M, 12 layers): 16 of its ragged sequences in one batch."""
    e, o = models(full_spec, synth.CONFIG_MIX[3], synth.CONFIG_SEED + 3)
    ids, mask = synth.config_inputs(3)
    ids, mask = ids[:16], mask[:16]
    check_exact(e.embed_padded(ids, mask), o.embed_batch(ids, mask), "exact c3 x16")


def test_exact_full_model_config4_all_rows(gpu, full_spec):
    """Config 4 at full size (B=256, L=128, 12 layers, Q8_0): all 256 rows bit-equal to the
    oracle's."""
    e, o = models(full_spec, "Q8_0", synth.CONFIG_SEED + 4)
    ids, mask = synth.config_inputs(4)
    check_exact(e.embed_padded(ids, mask), o.embed_batch(ids, mask), "exact c4 all rows")


def test_exact_mode_rejections_and_switch_back(gpu, small_spec):
    """F32 mode refuses the entries that cannot know each sequence's length; switching back to
    F16 gives the F16 rows again."""
    p = synth.model_path(small_spec, "Q8_0", 100)
    e = Embedder.load(p)
    m = e.model()
    ids = np.random.default_rng(9).integers(0, small_spec.vocab, 20).astype(np.int32)
    f16 = e.embed(ids)
    m.set_precision("f32")
    D = small_spec.d_model
    di, dm, dy = (_hip.DeviceBuffer.from_array(ids[None, :]), _hip.DeviceBuffer.from_array(np.ones((1, 20), np.int32)),
                  _hip.DeviceBuffer(D * 4))
    assert lib().lle_embed_batch_async(m.h, di.ptr, dm.ptr, 1, 20, D, dy.ptr, None) == -4
    off = _hip.DeviceBuffer.from_array(np.array([0, 20], np.int32))
    assert lib().lle_embed_packed_noalloc(m.h, di.ptr, off.ptr, 1, 20, 20, D, dy.ptr, None) == -4
    f32 = e.embed(ids)
    cos = float(np.dot(f16, f32) / np.linalg.norm(f16) / np.linalg.norm(f32))
    assert cos > 0.9999 and not np.array_equal(bits(f16), bits(f32))
    m.set_precision("f16")
    assert np.array_equal(bits(e.embed(ids)), bits(f16))
    assert lib().lle_model_set_precision(m.h, 7) == -1
    m.close()
