"""Concurrent use of one model from many host threads and streams.

The reference's TestEmbedConcurrentSafety (internal/embed/embedder_test.go:255-305) runs Embed
from 16 goroutines on one Embedder and checks every vector's dimension and unit norm. Here the
same load runs through the C ABI from 16 OS threads (ctypes releases the GIL for the call), mixing
lle_embed, lle_embed_batch and lle_embed_texts, and every row must equal, bit for bit, the row the
same call gives when run alone. Async calls on two caller streams, interleaved with host calls,
must not overlap on the model's workspace, and lle_last_error must stay per thread.
"""
import ctypes as C
import threading

import numpy as np
import pytest

from llmembed import Embedder, _hip, _lib, synth
from llmembed._lib import ptr

pytestmark = pytest.mark.gpu

N_THREADS = 16
CALLS = 5


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def emb(gpu, small_spec):
    return Embedder.load(synth.model_path(small_spec, "Q8_0", 100))


def workload(vocab):
    """Per thread, CALLS calls: id sequences of varying length, a small padded batch, texts."""
    rng = np.random.default_rng(77)
    work = []
    for t in range(N_THREADS):
        calls = []
        for c in range(CALLS):
            kind = (t + c) % 3
            if kind == 0:
                L = int(rng.integers(2, 200))
                calls.append(("ids", rng.integers(0, vocab, L).astype(np.int32)))
            elif kind == 1:
                B, L = int(rng.integers(2, 9)), int(rng.integers(4, 96))
                ids = rng.integers(0, vocab, (B, L)).astype(np.int32)
                lens = rng.integers(1, L + 1, B)
                mask = (np.arange(L)[None, :] < lens[:, None]).astype(np.int32)
                calls.append(("batch", (ids, mask)))
            else:
                calls.append(("texts", synth.texts(int(rng.integers(1, 12)), seed=1000 * t + c, max_words=60)))
        work.append(calls)
    return work


def run_call(e, call):
    kind, arg = call
    if kind == "ids":
        return e.embed(arg)[None, :]
    if kind == "batch":
        return e.embed_padded(*arg)
    return e.embed_texts(arg)


def test_sixteen_threads_bit_equal_to_serial(emb):
    work = workload(emb.model().vocab_size)
    serial = [[run_call(emb, c) for c in calls] for calls in work]
    print(f"serial: {sum(len(c) for c in work)} calls done", flush=True)
    got = [[None] * CALLS for _ in range(N_THREADS)]
    errors = []
    start = threading.Barrier(N_THREADS)

    def worker(t):
        try:
            start.wait()
            for c, call in enumerate(work[t]):
                got[t][c] = run_call(emb, call)
        except Exception as ex:  # reported below
            errors.append((t, repr(ex)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(N_THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=300)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors
    for t in range(N_THREADS):
        for c in range(CALLS):
            g, s = got[t][c], serial[t][c]
            assert g.shape == s.shape and g.shape[1] == emb.dim()
            assert np.all(np.isfinite(g))
            assert np.abs(np.linalg.norm(g.astype(np.float64), axis=1) - 1.0).max() < 1e-5
            assert np.array_equal(bits(g), bits(s)), (t, c, work[t][c][0])
    print(f"threads: {N_THREADS} x {CALLS} calls bit-equal to serial", flush=True)


def test_last_error_is_per_thread(emb):
    """Each thread fails with its own out-of-range id while the others succeed or fail; the
    message each thread reads names its own id."""
    lib = _lib.lib()
    vocab = emb.model().vocab_size
    barrier = threading.Barrier(N_THREADS)
    bad = []

    def worker(t):
        ids = np.array([101, 7, 102], np.int32)
        out = np.empty(emb.dim(), np.float32)
        for rep in range(3):
            barrier.wait()
            if t % 2 == 0:
                ids[1] = vocab + t  # invalid, distinct per thread
                rc = lib.lle_embed(emb.model().h, ptr(ids), None, 3, emb.dim(), ptr(out))
                barrier.wait()  # every odd thread has finished its successful call meanwhile
                msg = lib.lle_last_error().decode()
                if rc != -1 or f"token embedding {vocab + t}:" not in msg:
                    bad.append((t, rep, rc, msg))
            else:
                ids[1] = 7
                rc = lib.lle_embed(emb.model().h, ptr(ids), None, 3, emb.dim(), ptr(out))
                barrier.wait()
                msg = lib.lle_last_error().decode()
                if rc != 0 or "token embedding" in msg:
                    bad.append((t, rep, rc, msg))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(N_THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads)
    assert not bad, bad[:4]


def test_async_two_streams_interleaved_with_host_calls(emb):
    """Async forwards on two caller streams, host forwards between them, from two threads: every
    result equals the serial one bit for bit (forwards run on the model's stream; caller streams
    are joined by events, so no two forwards share the workspace at once)."""
    lib = _lib.lib()
    m = emb.model()
    rng = np.random.default_rng(5)
    D = emb.dim()
    cases = []
    for i in range(6):
        B, L = (4, 64) if i % 2 == 0 else (12, 128)  # 256 and 1536 tokens: both GEMM schedules
        ids = rng.integers(0, m.vocab_size, (B, L)).astype(np.int32)
        mask = np.ones((B, L), np.int32)
        cases.append((ids, mask))
    serial = [emb.embed_padded(ids, mask) for ids, mask in cases]
    host_ids = rng.integers(0, m.vocab_size, 40).astype(np.int32)
    host_ref = emb.embed(host_ids)

    streams = [_hip.Stream(), _hip.Stream()]
    dev = []
    for ids, mask in cases:
        B, L = ids.shape
        dev.append((_hip.DeviceBuffer.from_array(ids), _hip.DeviceBuffer.from_array(mask), _hip.DeviceBuffer(B * D * 4)))
    errors = []

    def worker(w):
        try:
            s = streams[w]
            for rep in range(3):
                for i in range(w, len(cases), 2):
                    B, L = cases[i][0].shape
                    di, dm, do = dev[i]
                    rc = lib.lle_embed_batch_async(m.h, C.c_void_p(di.value), C.c_void_p(dm.value), B, L, D,
                                                   C.c_void_p(do.value), s.h)
                    if rc:
                        errors.append((w, rc, lib.lle_last_error().decode()))
                    h = emb.embed(host_ids)  # host call while async work is queued
                    if not np.array_equal(bits(h), bits(host_ref)):
                        errors.append((w, rep, "host row differs"))
                s.synchronize()
                for i in range(w, len(cases), 2):
                    B, _ = cases[i][0].shape
                    got = dev[i][2].download((B, D), np.float32)
                    if not np.array_equal(bits(got), bits(serial[i])):
                        errors.append((w, rep, i, "async rows differ"))
        except Exception as ex:
            errors.append((w, repr(ex)))

    threads = [threading.Thread(target=worker, args=(w,)) for w in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=300)
    assert not any(th.is_alive() for th in threads)
    assert not errors, errors[:4]
