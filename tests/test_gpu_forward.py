"""GPU parity of the whole encoder forward (Embed / EmbedBatch) against the CPU oracle.

Bar (from the task's north star): per-vector cosine >= 0.9999 and max-abs <= 1e-3 on the final
L2-normalised embeddings, on the same seeded synthetic GGUF models and token ids. EmbedBatch
rows must equal Embed bit for bit (internal/embed/embedder_test.go:116-145,212-253).
"""
import numpy as np
import pytest

import oracle
from llmembed import Embedder, LLEError, synth

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999
MAXABS = 1e-3


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def compare(got, ref, what):
    got = np.atleast_2d(got).astype(np.float64)
    ref = np.atleast_2d(ref).astype(np.float64)
    cos = np.sum(got * ref, axis=1) / np.linalg.norm(got, axis=1) / np.linalg.norm(ref, axis=1)
    mx = float(np.abs(got - ref).max())
    print(f"{what}: min cos {cos.min():.7f}  max abs {mx:.2e}", flush=True)
    assert cos.min() >= COS_MIN, (what, cos.min())
    assert mx <= MAXABS, (what, mx)


_models = {}


def models(spec, mix, seed=100, qkv_std=0.02):
    key = (spec, mix, seed, qkv_std)
    if key not in _models:
        p = synth.model_path(spec, mix, seed, qkv_std)
        _models[key] = (Embedder.load(p), oracle.OracleModel(p))
    return _models[key]


@pytest.mark.parametrize("mix", ["Q8_0", "Q4_K", "Q5_K", "Q6_K", "F32", "Q4_K_M", "Q5_K_M"])
def test_embed_small_model(gpu, small_spec, mix):
    e, o = models(small_spec, mix)
    rng = np.random.default_rng(21)
    for L in (8, 45, 128):
        ids = rng.integers(0, small_spec.vocab, L).astype(np.int32)
        compare(e.embed(ids), o.embed(ids), f"{mix} L={L}")


@pytest.mark.parametrize("mix", ["Q8_0", "Q4_K", "Q5_K", "Q6_K", "F32", "Q5_K_M"])
def test_large_batch_formats(gpu, small_spec, mix):
    """A batch of >= 1024 packed rows (12 sequences of ragged length, host entry) runs the
    large-batch GEMMs on the resident f16 weight copies: QKV on 256 x 256 tiles with its RoPE
    operands staged in LDS (row positions through the packed-row map), up||gate, down and the
    full-row out projection. Every row equals the sequence embedded alone (the small-batch
    schedule) bit for bit, and the rows match the oracle."""
    e, o = models(small_spec, mix)
    rng = np.random.default_rng(61)
    B, L = 12, 128
    ids = rng.integers(0, small_spec.vocab, (B, L)).astype(np.int32)
    lens = rng.integers(88, L + 1, B)
    lens[0] = L
    mask = np.zeros((B, L), np.int32)
    for b in range(B):
        mask[b, :lens[b]] = 1
    print(f"large batch {mix}: {int(lens.sum())} rows", flush=True)
    assert lens.sum() >= 1024
    batch = e.embed_padded(ids, mask)
    for b in (0, 5, 11):
        assert np.array_equal(bits(e.embed(ids[b, :lens[b]])), bits(batch[b])), (mix, b)
    compare(batch, o.embed_batch(ids, mask), f"large batch {mix}")


def test_config1_full_model(gpu, full_spec):
    """Config 1: full 12-layer Q8_0 model, B=1, L=8."""
    e, o = models(full_spec, "Q8_0", synth.CONFIG_SEED + 1)
    ids, mask = synth.config_inputs(1)
    compare(e.embed(ids[0]), o.embed(ids[0]), "c1")


@pytest.mark.parametrize("mix", ["Q8_0", "Q6_K", "Q5_K_M"])
def test_config4_full_size(gpu, full_spec, mix):
    """Config 4 at its full size on each of its three formats (full 12-layer model, B=256,
    L=128: the 32768-token schedule of the benchmark). Every one of the 256 rows matches the
    oracle (cosine and max-abs, the reference's per-vector contract,
    internal/embed/embedder_test.go:116-145); rows are finite with unit norm; a second run gives
    the same bits; and rows equal the same sequences embedded alone (the <= 64-token schedule:
    split-K small GEMMs, fused LayerNorm prologues, 64-query attention) bit for bit."""
    e, o = models(full_spec, mix, synth.CONFIG_SEED + 4)
    ids, mask = synth.config_inputs(4)
    assert ids.shape == (256, 128) and int(mask.sum()) == 256 * 128
    batch = e.embed_padded(ids, mask)
    assert batch.shape == (256, full_spec.d_model) and np.all(np.isfinite(batch))
    norms = np.linalg.norm(batch.astype(np.float64), axis=1)
    assert np.abs(norms - 1.0).max() < 1e-5, np.abs(norms - 1.0).max()
    assert np.array_equal(bits(e.embed_padded(ids, mask)), bits(batch))
    for i in (0, 77, 255):
        assert np.array_equal(bits(e.embed(ids[i])), bits(batch[i])), i
    print(f"c4 {mix}: oracle on all 256 rows", flush=True)
    compare(batch, o.embed_batch(ids, mask), f"c4 full size {mix}, all rows")


def test_config3_full_size(gpu, full_spec):
    """Config 3 at its full size (full 12-layer Q4_K_M model: Q4_K / Q5_K / Q6_K projections,
    B=64, lengths in [16, 128] padded to 128): every row matches the oracle; rows are finite
    with unit norm and equal each sequence embedded alone bit for bit."""
    e, o = models(full_spec, synth.CONFIG_MIX[3], synth.CONFIG_SEED + 3)
    ids, mask = synth.config_inputs(3)
    B, L = ids.shape
    lens = mask.sum(axis=1)
    assert (B, L) == (64, 128)
    batch = e.embed_padded(ids, mask)
    assert np.all(np.isfinite(batch))
    assert np.abs(np.linalg.norm(batch.astype(np.float64), axis=1) - 1.0).max() < 1e-5
    picks = sorted({int(np.argmin(lens)), int(np.argmax(lens)), 31})
    for i in picks:
        assert np.array_equal(bits(e.embed(ids[i, :lens[i]])), bits(batch[i])), i
    compare(batch, o.embed_batch(ids, mask), "c3 full size, all rows")


def test_config5_full_size(gpu, full_spec):
    """Config 5 at its full size (full 12-layer Q8_0 model, B=8, lengths in [1024, 2048] padded
    to 2048): finite unit-norm rows, rows equal each sequence embedded alone bit for bit, and the
    shortest, the longest and a middle sequence match the oracle (all eight take the scalar
    oracle over a minute)."""
    e, o = models(full_spec, "Q8_0", synth.CONFIG_SEED + 5)
    ids, mask = synth.config_inputs(5)
    B, L = ids.shape
    lens = mask.sum(axis=1)
    assert (B, L) == (8, 2048) and lens.min() >= 1024
    batch = e.embed_padded(ids, mask)
    assert np.all(np.isfinite(batch))
    assert np.abs(np.linalg.norm(batch.astype(np.float64), axis=1) - 1.0).max() < 1e-5
    order = np.argsort(lens)
    picks = sorted({int(order[0]), int(order[-1]), int(order[B // 2])})
    for i in picks:
        assert np.array_equal(bits(e.embed(ids[i, :lens[i]])), bits(batch[i])), i
    print(f"c5: oracle on rows {picks} (lengths {[int(lens[i]) for i in picks]})", flush=True)
    compare(batch[picks], o.embed_batch(ids[picks], mask[picks]), "c5 full size")


def test_hidden_states(gpu, small_spec):
    e, o = models(small_spec, "Q8_0")
    ids = np.random.default_rng(3).integers(0, small_spec.vocab, 33).astype(np.int32)
    h = e.model().forward(ids)
    ref = o.forward(ids)
    err = np.abs(h - ref)
    print("hidden max abs", err.max(), "rms", np.sqrt(np.mean(err ** 2)))
    assert np.sqrt(np.mean(err.astype(np.float64) ** 2)) < 1e-2
    cos = np.sum(h * ref, axis=1) / np.linalg.norm(h, axis=1) / np.linalg.norm(ref, axis=1)
    assert cos.min() > 0.9999


def test_batch_invariance(gpu, small_spec):
    """EmbedBatch rows == Embed of each row, bit for bit, for mixed lengths and padding."""
    e, _ = models(small_spec, "Q4_K_M")
    rng = np.random.default_rng(5)
    lens = [1, 7, 8, 64, 65, 100, 130, 3]
    seqs = [rng.integers(0, small_spec.vocab, n).astype(np.int32) for n in lens]
    batch = e.embed_batch(seqs)
    for s, b in zip(seqs, batch):
        assert np.array_equal(bits(e.embed(s)), bits(b)), len(s)
    # the same rows inside a larger padded batch
    big = e.embed_batch(seqs + seqs[::-1] + [rng.integers(0, small_spec.vocab, 200).astype(np.int32)])
    for i in range(len(seqs)):
        assert np.array_equal(bits(big[i]), bits(batch[i]))


@pytest.mark.parametrize("mix", ["Q8_0", "Q5_K", "Q6_K", "F32", "Q4_K_M"])
def test_full_row_layernorm_path_bitexact(gpu, small_spec, mix):
    """Batches of >= 1024 tokens run the attention output projection as a full-row GEMM with
    the residual + LayerNorm in its epilogue; each row must equal the same sequence embedded
    alone (128-token tiles + separate LayerNorm kernel), bit for bit, and match the oracle."""
    e, o = models(small_spec, mix)
    rng = np.random.default_rng(44)
    seqs = [rng.integers(0, small_spec.vocab, n).astype(np.int32) for n in (128, 97, 128, 64, 128, 128, 5, 128, 128)]
    batch = e.embed_batch(seqs)  # 9 x 128 = 1152 padded tokens
    for s, b in zip(seqs, batch):
        assert np.array_equal(bits(e.embed(s)), bits(b)), len(s)
    compare(batch[1], o.embed(seqs[1]), f"{mix} full-row LN")


@pytest.mark.parametrize("mix", ["Q8_0", "Q4_K_M"])
def test_decoding_gemm_path_matches_f16_copy_path(gpu, small_spec, mix, monkeypatch):
    """Without the resident f16 weight copy (LLE_NO_F16_COPY=1) the >= 1024-token GEMMs decode
    the quantised planes in their loop; the embeddings must equal the f16-copy path's bit for
    bit (same operands, same MFMA order)."""
    p = synth.model_path(small_spec, mix, 100, 0.02)
    rng = np.random.default_rng(45)
    ids = rng.integers(0, small_spec.vocab, (12, 100)).astype(np.int32)
    mask = np.ones_like(ids)
    mask[3, 70:] = 0
    ref = models(small_spec, mix)[0].embed_padded(ids, mask)
    monkeypatch.setenv("LLE_NO_F16_COPY", "1")
    e = Embedder.load(p)
    try:
        got = e.embed_padded(ids, mask)
    finally:
        e.model().close()
    assert np.array_equal(bits(got), bits(ref))


def test_padded_batch_vs_oracle(gpu, small_spec):
    """Config-3 style: right-padded batch with per-row lengths, Q4_K_M."""
    e, o = models(small_spec, "Q4_K_M")
    ids, mask = synth.config_inputs(3)
    ids, mask = ids[:16], mask[:16]
    compare(e.embed_padded(ids, mask), o.embed_batch(ids, mask), "c3-style B=16")


def test_arbitrary_mask(gpu, small_spec):
    """Interior zeros in the mask: keys masked in attention, rows excluded from pooling."""
    e, o = models(small_spec, "Q8_0")
    rng = np.random.default_rng(6)
    ids = rng.integers(0, small_spec.vocab, 70).astype(np.int32)
    mask = np.ones(70, np.int32)
    mask[[0, 5, 33, 64, 69]] = 0
    compare(e.embed(ids, mask), o.embed(ids, mask), "interior mask")


def test_matryoshka(gpu, small_spec):
    e, o = models(small_spec, "Q8_0")
    ids = np.random.default_rng(8).integers(0, small_spec.vocab, 20).astype(np.int32)
    for d in (512, 256, 64):
        e.set_target_dim(d)
        try:
            v = e.embed(ids)
        finally:
            e.set_target_dim(768)
        assert v.shape == (d,) and abs(float(np.linalg.norm(v.astype(np.float64))) - 1) < 1e-5
        compare(v, o.embed(ids, out_dim=d), f"matryoshka {d}")


def test_small_forward_pool_paths(gpu, small_spec):
    """Forwards of <= 16 tokens end in one kernel (last LayerNorm + mean-pool + L2, rows kept in
    LDS). Mask holes, several packed sequences and Matryoshka widths through it must equal the
    same rows inside a larger batch (separate LayerNorm and pool kernels) bit for bit, and
    match the oracle."""
    e, o = models(small_spec, "Q8_0")
    rng = np.random.default_rng(17)
    long_row = rng.integers(0, small_spec.vocab, 40).astype(np.int32)

    def in_big_batch(ids, mask):  # the rows again, beside a 40-token sequence (> 16 tokens)
        B, L = ids.shape
        big_ids = np.zeros((B + 1, 40), np.int32)
        big_mask = np.zeros((B + 1, 40), np.int32)
        big_ids[:B, :L], big_mask[:B, :L] = ids, mask
        big_ids[B], big_mask[B] = long_row, 1
        return e.embed_padded(big_ids, big_mask)[:B]

    # one sequence with mask holes (first, interior and last positions)
    ids = rng.integers(0, small_spec.vocab, (1, 12)).astype(np.int32)
    mask = np.ones((1, 12), np.int32)
    mask[0, [0, 5, 11]] = 0
    small = e.embed_padded(ids, mask)
    assert np.array_equal(bits(small), bits(in_big_batch(ids, mask)))
    compare(small[0], o.embed(ids[0], mask[0]), "small forward, mask holes")
    # three sequences packed into 12 tokens, right-padded to 6
    lens = [3, 5, 4]
    ids = rng.integers(0, small_spec.vocab, (3, 6)).astype(np.int32)
    mask = (np.arange(6)[None, :] < np.array(lens)[:, None]).astype(np.int32)
    small = e.embed_padded(ids, mask)
    assert np.array_equal(bits(small), bits(in_big_batch(ids, mask)))
    for b, n in enumerate(lens):
        compare(small[b], o.embed(ids[b, :n]), f"small forward, packed row {b}")
    # Matryoshka widths
    ids = rng.integers(0, small_spec.vocab, (1, 10)).astype(np.int32)
    mask = np.ones((1, 10), np.int32)
    for d in (256, 64):
        e.set_target_dim(d)
        try:
            small = e.embed_padded(ids, mask)
            big = in_big_batch(ids, mask)
        finally:
            e.set_target_dim(768)
        assert small.shape == (1, d) and np.array_equal(bits(small), bits(big)), d
        compare(small[0], o.embed(ids[0], out_dim=d), f"small forward, matryoshka {d}")


def test_cutoff_active_attention(gpu, small_spec):
    """Large attention logits (qkv weights N(0, 0.3)): the softmax's x < -10 cutoff drops keys,
    exercising the kernel's fixed-max second pass."""
    e, o = models(small_spec, "Q8_0", 101, qkv_std=0.3)
    rng = np.random.default_rng(12)
    for L in (16, 96, 300):
        ids = rng.integers(0, small_spec.vocab, L).astype(np.int32)
        compare(e.embed(ids), o.embed(ids), f"cutoff L={L}")


def test_long_sequence(gpu, small_spec):
    """Config-5 style long context on the 2-layer model (L = 1100 and 2048)."""
    e, o = models(small_spec, "Q8_0")
    rng = np.random.default_rng(13)
    for L in (1100, 2048):
        ids = rng.integers(0, small_spec.vocab, L).astype(np.int32)
        compare(e.embed(ids), o.embed(ids), f"long L={L}")


def test_sliced_pool_bitexact(gpu, small_spec):
    """Few long rows (B <= 64, padded L >= 512) are mean-pooled by D/64 column-slice blocks,
    other batches by one block per sequence (and <= 64 tokens inside the last LayerNorm kernel).
    Every form sums each column over the kept rows in row order, so a sequence's embedding has
    the same bits whichever form pools it: lengths on both sides of the rule embedded alone,
    padded together to L = 1100 (sliced), and in a batch of 68 rows of that length (row form)."""
    e, o = models(small_spec, "Q8_0")
    rng = np.random.default_rng(14)
    lens = [300, 513, 40, 1000]
    seqs = [rng.integers(0, small_spec.vocab, n).astype(np.int32) for n in lens]
    alone = [e.embed(s) for s in seqs]
    L = 1100
    ids = np.zeros((len(lens), L), np.int32)
    mask = np.zeros((len(lens), L), np.int32)
    for i, s in enumerate(seqs):
        ids[i, : len(s)] = s
        mask[i, : len(s)] = 1
    batch = e.embed_padded(ids, mask)
    many = e.embed_padded(np.tile(ids, (17, 1)), np.tile(mask, (17, 1)))
    for i in range(len(lens)):
        assert np.array_equal(bits(batch[i]), bits(alone[i])), lens[i]
        assert np.array_equal(bits(many[i]), bits(alone[i])), lens[i]
        assert np.array_equal(bits(many[4 * 16 + i]), bits(alone[i])), lens[i]
    compare(batch[1], o.embed(seqs[1]), "sliced pool L=513")


def test_errors(gpu, small_spec):
    e, _ = models(small_spec, "Q8_0")
    with pytest.raises(LLEError):
        e.embed(np.array([101, small_spec.vocab, 102], np.int32))
    with pytest.raises(LLEError):
        e.embed(np.zeros(small_spec.ctx + 1, np.int32))
    with pytest.raises(LLEError):
        Embedder.load("/nonexistent/model.gguf")


def test_graph_replay_matches_eager(gpu, small_spec):
    """Small forwards replay a captured HIP graph. Every replay, interleaved with other shapes
    and with eager (large, and timing-mode) forwards, must equal the eager result bit for bit."""
    e, o = models(small_spec, "Q8_0")
    rng = np.random.default_rng(31)
    a = rng.integers(0, small_spec.vocab, 8).astype(np.int32)
    b = rng.integers(0, small_spec.vocab, 21).astype(np.int32)
    big_ids = rng.integers(0, small_spec.vocab, (40, 128)).astype(np.int32)
    m = e.model()
    m.set_timing(True)  # timed forwards run eagerly
    ea, eb = e.embed(a), e.embed(b)
    m.set_timing(False)
    big = e.embed_padded(big_ids, np.ones_like(big_ids))  # 5120 tokens: eager
    for _ in range(5):
        assert np.array_equal(bits(e.embed(a)), bits(ea))
        assert np.array_equal(bits(e.embed(b)), bits(eb))
        assert np.array_equal(bits(e.embed_padded(big_ids, np.ones_like(big_ids))), bits(big))
    compare(e.embed(a), o.embed(a), "graph replay")


def test_single_class_timing(gpu, small_spec):
    """lle_model_set_timing_kernel brackets only one kernel class, with no synchronisation per
    forward: its totals hold exactly that class's launches (one per layer per forward) and the
    rows equal untimed forwards bit for bit."""
    e, _ = models(small_spec, "Q8_0")
    rng = np.random.default_rng(37)
    ids = rng.integers(0, small_spec.vocab, (40, 128)).astype(np.int32)  # 5120 tokens: eager
    m = e.model()
    ref = e.embed_padded(ids, np.ones_like(ids))
    m.set_timing_kernel("gemm_upgate")
    outs = [e.embed_padded(ids, np.ones_like(ids)) for _ in range(3)]
    kt = m.timing()
    m.set_timing_kernel(None)
    assert set(kt) == {"gemm_upgate"}
    assert kt["gemm_upgate"]["launches"] == 3 * small_spec.n_layer
    assert kt["gemm_upgate"]["total_ms"] > 0
    for o_ in outs:
        assert np.array_equal(bits(o_), bits(ref))
    m.set_timing(True)
    e.embed_padded(ids, np.ones_like(ids))
    kt = m.timing()
    m.set_timing(False)
    assert {"gemm_qkv", "attention", "gemm_upgate"} <= set(kt)


@pytest.mark.parametrize("B,L,seed", [(3, 8, 1), (4, 20, 2), (5, 40, 3), (12, 100, 4), (20, 128, 5)])
def test_packed_rows_equal_padded_forward(gpu, small_spec, B, L, seed):
    """lle_embed_batch (host pointers) drops the positions after each row's last valid token;
    lle_embed_batch_async (device pointers) computes every position. The embeddings must agree
    bit for bit, across the small fused (<= 16 rows), split-K (<= 64), decoding (< 1024) and
    LDS-DMA (>= 1024) GEMM paths that the two row counts select."""
    from llmembed import _hip
    from llmembed._lib import check, lib

    e, o = models(small_spec, "Q8_0")
    D = small_spec.d_model
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, small_spec.vocab, (B, L)).astype(np.int32)
    mask = np.zeros((B, L), np.int32)
    for b in range(B):
        mask[b, :int(rng.integers(1, L + 1))] = 1
    mask[0, :] = 0                      # no valid token: kept whole (uniform softmax over L keys)
    mask[1, :] = 1                      # no padding
    mask[2, :] = 0                      # interior zeros, valid token at the end of a long gap
    mask[2, [0, L // 2, L - 2]] = 1
    print(f"packed: B={B} L={L} rows {int(sum(L if not r.any() else np.nonzero(r)[0][-1] + 1 for r in mask))}"
          f" of {B * L}", flush=True)
    host = e.embed_padded(ids, mask)
    di, dm = _hip.DeviceBuffer.from_array(ids), _hip.DeviceBuffer.from_array(mask)
    do = _hip.DeviceBuffer(B * D * 4)
    check(lib().lle_embed_batch_async(e.model().h, di.ptr, dm.ptr, B, L, D, do.ptr, None))
    _hip.synchronize()
    dev = do.download((B, D), np.float32)
    assert np.array_equal(bits(host), bits(dev))
    compare(host[1:], o.embed_batch(ids[1:], mask[1:]), f"packed B={B} L={L}")


@pytest.mark.parametrize("B,last", [(188, 64), (260, 37)])
def test_ragged_large_batch_tiles(gpu, small_spec, B, last):
    """Packed row counts that leave the large-batch tiles partly past the last row: 24,000 rows
    (256 x 288 QKV tiles, the last 256-row tile 64 rows short) and 33,189 rows (the 128-row
    full-row out projection's last block 91 rows short, and partial last 256-row tiles of the
    down and up||gate GEMMs). Rows of sequences at the start, middle and end of the batch equal the same
    sequences embedded alone bit for bit, and match the oracle."""
    e, o = models(small_spec, "Q8_0")
    L = 128
    rng = np.random.default_rng(B)
    ids = rng.integers(0, small_spec.vocab, (B, L)).astype(np.int32)
    mask = np.ones((B, L), np.int32)
    mask[-1, last:] = 0
    print(f"ragged: B={B} rows {int(mask.sum())}", flush=True)
    batch = e.embed_padded(ids, mask)
    assert np.all(np.isfinite(batch))
    for i in (0, B // 2, B - 2, B - 1):
        n = int(mask[i].sum())
        assert np.array_equal(bits(e.embed(ids[i, :n])), bits(batch[i])), i
    compare(batch[[0, B - 1]], o.embed_batch(ids[[0, B - 1]], mask[[0, B - 1]]), f"ragged B={B}")


def test_key_tile_boundaries(gpu, small_spec):
    """Sequences whose last stored key falls exactly on, just past, and well inside a 64-key
    tile (lengths 64, 128, 65, 192 and 1 in a batch padded to 192): the attention reads K tiles
    bounded at that key and zeroes V^T's columns only in the tile that holds it. The padded
    device entry (every position stored), the packed host entry (positions past each sequence's
    last valid token dropped) and single-sequence embeds agree bit for bit, and match the
    oracle."""
    from llmembed import _hip
    from llmembed._lib import check, lib

    e, o = models(small_spec, "Q8_0")
    D = small_spec.d_model
    lens = [64, 128, 65, 192, 1]
    B, L = len(lens), 192
    rng = np.random.default_rng(53)
    ids = rng.integers(0, small_spec.vocab, (B, L)).astype(np.int32)
    mask = np.zeros((B, L), np.int32)
    for b, n in enumerate(lens):
        mask[b, :n] = 1
    print(f"key tiles: lengths {lens} padded to {L}", flush=True)
    host = e.embed_padded(ids, mask)
    di, dm = _hip.DeviceBuffer.from_array(ids), _hip.DeviceBuffer.from_array(mask)
    do = _hip.DeviceBuffer(B * D * 4)
    check(lib().lle_embed_batch_async(e.model().h, di.ptr, dm.ptr, B, L, D, do.ptr, None))
    _hip.synchronize()
    dev = do.download((B, D), np.float32)
    assert np.array_equal(bits(host), bits(dev))
    for b, n in enumerate(lens):
        assert np.array_equal(bits(e.embed(ids[b, :n])), bits(host[b])), lens[b]
    compare(host, o.embed_batch(ids, mask), "key tile boundaries")


@pytest.mark.parametrize("qkv_std", [0.02, 0.3])
def test_small_batch_schedule_bitexact(gpu, small_spec, qkv_std):
    """Batches of <= 16 rows run the small-batch schedule (LayerNorms inside the consuming GEMMs,
    split-K partials, one-tile attention); larger batches the general one. A row must come out
    with the same bits either way, with masked keys inside the sequence, padding, a sequence with
    no valid token and (qkv_std 0.3) the x < -10 cutoff dropping keys."""
    e, o = models(small_spec, "Q8_0", 101 if qkv_std != 0.02 else 100, qkv_std=qkv_std)
    rng = np.random.default_rng(41)
    V = small_spec.vocab
    cases = []
    for L in (1, 5, 12, 16):
        ids = rng.integers(0, V, L).astype(np.int32)
        cases.append((ids, np.ones(L, np.int32)))
    ids = rng.integers(0, V, 14).astype(np.int32)
    cases.append((ids, np.array([1, 1, 0, 1, 0, 0, 1, 1, 1, 0, 1, 1, 0, 0], np.int32)))  # interior + trailing zeros
    cases.append((rng.integers(0, V, 6).astype(np.int32), np.zeros(6, np.int32)))  # no valid token
    filler = rng.integers(0, V, (2, 40)).astype(np.int32)
    for ids, mask in cases:
        L = ids.size
        print(f"small batch: L={L} valid={int(mask.sum())} qkv_std={qkv_std}", flush=True)
        small = e.embed_padded(ids[None, :], mask[None, :])      # <= 16 rows
        big_ids = np.zeros((3, 40), np.int32)
        big_mask = np.zeros((3, 40), np.int32)
        big_ids[0, :L], big_mask[0, :L] = ids, mask
        big_ids[1:], big_mask[1:] = filler, 1
        big = e.embed_padded(big_ids, big_mask)                  # > 16 rows
        assert np.array_equal(bits(small[0]), bits(big[0])), (L, mask.tolist())
        if mask.any():
            compare(small, o.embed_batch(ids[None, :], mask[None, :]), f"small batch L={L}")


def test_packed_device_entry(gpu, small_spec):
    """lle_embed_packed_async: sequences back to back on the device (no padding stored or
    computed) give the rows of the padded host entry bit for bit; an inconsistent offset table is
    made safe and reported in the status word (bit 2)."""
    import ctypes as C

    from llmembed import _hip
    from llmembed._lib import check, lib

    e, o = models(small_spec, "Q8_0")
    m = e.model()
    D, V = small_spec.d_model, small_spec.vocab
    rng = np.random.default_rng(77)
    for lens in ([8], [1, 5, 16], [100, 3, 64, 1, 77], [300] * 6):
        B, L = len(lens), max(lens)
        seqs = [rng.integers(0, V, n).astype(np.int32) for n in lens]
        ids = np.zeros((B, L), np.int32)
        mask = np.zeros((B, L), np.int32)
        for b, sq in enumerate(seqs):
            ids[b, :sq.size], mask[b, :sq.size] = sq, 1
        ref = e.embed_padded(ids, mask)
        packed = np.concatenate(seqs)
        off = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        print(f"packed device entry: lens={lens}", flush=True)
        di, do_, dy = _hip.DeviceBuffer.from_array(packed), _hip.DeviceBuffer.from_array(off), _hip.DeviceBuffer(B * D * 4)
        check(lib().lle_embed_packed_async(m.h, di.ptr, do_.ptr, B, int(packed.size), L, D, dy.ptr, None))
        _hip.synchronize()
        assert np.array_equal(bits(dy.download((B, D), np.float32)), bits(ref)), lens
        st = C.c_int32(-1)
        check(lib().lle_model_status(m.h, C.byref(st)))
        assert st.value == 0
    # offsets that decrease and overrun T: clamped on the device, flagged, no fault
    packed = rng.integers(0, V, 9).astype(np.int32)
    di, do_, dy = (_hip.DeviceBuffer.from_array(packed), _hip.DeviceBuffer.from_array(np.array([0, 5, 3, 12], np.int32)),
                   _hip.DeviceBuffer(3 * D * 4))
    e.embed_padded(packed[None, :], np.ones((1, 9), np.int32))  # a host call clears the status word
    check(lib().lle_embed_packed_async(m.h, di.ptr, do_.ptr, 3, 9, 9, D, dy.ptr, None))
    _hip.synchronize()
    st = C.c_int32(-1)
    check(lib().lle_model_status(m.h, C.byref(st)))
    assert st.value & 2
