"""EmbedBatch / Embed over text (internal/embed/embedder.go:46-133) through lle_embed_texts:
the library's native tokeniser feeds length-ordered, padded GPU batches. Each row must equal,
bit for bit, lle_embed of the oracle tokenisation of TaskPrefix + text (Encode,
internal/embed/tokenizer.go:47-78, with max_len = context_length), whatever the batching.
"""
import numpy as np
import pytest

import wordpiece as wp
from llmembed import Embedder, synth

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def emb(gpu, small_spec):
    return Embedder.load(synth.model_path(small_spec, "Q8_0", 100))


@pytest.fixture(scope="module")
def otok(small_spec):
    return wp.Tokenizer(wp.read_gguf_string_array(synth.model_path(small_spec, "Q8_0", 100), "tokenizer.ggml.tokens"))


def corpus():
    t = synth.texts(60, seed=31, min_words=0, max_words=150)
    long = " ".join(synth.texts(1, seed=32, min_words=2600, max_words=2600))  # > 2048 tokens: truncated
    return t + ["", "Hello, World!", "  \t ", long, "naïve café — 中文 🙂", b"bad \xff\xfe utf-8"]


def test_embed_texts_equals_embed_of_oracle_ids(emb, otok):
    texts = corpus()
    print(f"embed_texts: {len(texts)} texts", flush=True)
    out = emb.embed_texts(texts)
    ctx = emb.model().max_seq_len
    assert out.shape == (len(texts), emb.dim())
    for i, t in enumerate(texts):
        tb = t if isinstance(t, bytes) else t.encode()
        ids = otok.encode(emb.task_prefix.encode() + tb, ctx)
        if i == len(texts) - 3:
            assert len(ids) == ctx and ids[-1] == 102
        ref = emb.embed(np.array(ids, np.int32))
        assert np.array_equal(bits(out[i]), bits(ref)), (i, len(ids))


def test_embed_texts_batching_invariance(emb):
    texts = corpus()[:-3]
    a = emb.embed_texts(texts)
    b = emb.embed_texts(texts, max_batch_tokens=300)   # many small batches
    c = emb.embed_texts(texts[::-1])[::-1]             # other order, other batch composition
    assert np.array_equal(bits(a), bits(b))
    assert np.array_equal(bits(a), bits(c))
    one = emb.embed(texts[5])                          # Embed(text)
    assert np.array_equal(bits(one), bits(a[5]))
    lst = emb.embed_batch(texts[:7])                   # EmbedBatch(texts)
    assert np.array_equal(bits(np.stack(lst)), bits(a[:7]))


def test_embed_texts_matryoshka_and_prefix(emb):
    texts = synth.texts(9, seed=33)
    full = emb.embed_texts(texts)
    try:
        emb.set_target_dim(128)
        short = emb.embed_texts(texts)
        emb.task_prefix = "search_document: "
        doc = emb.embed_texts(texts)
        ref = np.stack([emb.embed(wp_ids) for wp_ids in
                        (emb.tokenizer.encode("search_document: " + t, emb.model().max_seq_len)[0] for t in texts)])
    finally:
        emb.set_target_dim(emb.model().hidden_dim)
        emb.task_prefix = "search_query: "
    assert short.shape == (9, 128)
    n = np.linalg.norm(full[:, :128].astype(np.float64), axis=1, keepdims=True)
    np.testing.assert_allclose(short, full[:, :128] / n, rtol=0, atol=2e-6)
    assert np.array_equal(bits(doc), bits(ref))
    assert not np.array_equal(bits(doc), bits(short))
