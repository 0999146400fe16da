#!/usr/bin/env python3
"""Benchmark of the MI355X encoder forward (one JSON line on stdout).

Headline workload (BASELINE.json metric "embeddings/sec at B=256,L=128 Q8_0"): config 4 —
full 12-layer nomic-bert, random-init N(0, 0.02) Q8_0 GGUF, B=256 sequences of L=128 tokens,
every position valid. A step = one batched forward (embedding gather ... mean-pool + L2) over
the batch, with ids/mask already resident in HBM and the embeddings left in HBM.

Also reported: p50/p90 device latency of config 1 (B=1, L=8; HIP events, weights rotated over
three model copies so they stream from HBM) with its HBM roofline fraction, per-kernel
HIP-event times, the dominant kernel's roofline fraction (measured live with HIP events on
the stream the kernels run on) and the CPU oracle's embeddings/s on a bounded sample of the
same workload, timed on this host.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "llm-embed_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "encoder_c4_q8_0_hbm_traffic.md")


def committed_traffic(scope):
    """HBM bytes per launch of a kernel scope, from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE passes, each scaled by its calibration copy). None if absent."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 6 and cells[0] == scope:
                    return int(cells[4].replace(",", "")), os.path.relpath(TRAFFIC_PROFILE, ROOT)
    except OSError:
        pass
    return None, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--latency-iters", type=int, default=200)
    ap.add_argument("--cpu-seqs", type=int, default=256, help="sequences in the CPU-baseline sample (0 = skip)")
    ap.add_argument("--mix", default="Q8_0")
    ap.add_argument("--no-extras", dest="extras", action="store_false",
                    help="skip the config-3 / config-5 / other-quantisation runs")
    ap.add_argument("--probe-traffic", action="store_true",
                    help="for rocprofv3 --pmc runs: two config-4 forwards, then one 256 MiB device-to-device copy "
                         "(the calibration of FETCH_SIZE / WRITE_SIZE); prints no JSON")
    ap.add_argument("--probe-config", type=int, default=4, choices=(1, 3, 4, 5),
                    help="with --probe-traffic: the configuration whose two forwards are run (padded batch, "
                         "device-pointer entry); config 1 runs 30 forwards rotated over three model copies "
                         "(the cold-MALL latency setting) after 30 warm-ups")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); sequences are "
              "independent, so N GPUs would each run this same workload on B/N sequences.", file=sys.stderr)
        sys.exit(2)

    import llmembed
    from llmembed import _hip, synth
    from llmembed._lib import check, lib

    llmembed.init(0)
    log = lambda *a: print(*a, file=sys.stderr, flush=True)  # noqa: E731
    spec = synth.ModelSpec()
    path = synth.model_path(spec, args.mix, synth.CONFIG_SEED + 4)
    log(f"[bench] model {os.path.basename(path)}")
    emb = llmembed.Embedder.load(path)
    model = emb.model()
    L_ = lib()

    # ---------------------------------------------------------------- config 4 throughput
    ids, mask = synth.config_inputs(4)
    B, L = ids.shape
    D = model.hidden_dim
    d_ids, d_mask = _hip.DeviceBuffer.from_array(ids), _hip.DeviceBuffer.from_array(mask)
    d_out = _hip.DeviceBuffer(B * D * 4)
    stream = _hip.Stream()

    def step():
        check(L_.lle_embed_batch_async(model.h, d_ids.ptr, d_mask.ptr, B, L, D, d_out.ptr, stream.h))

    if args.probe_traffic:
        if args.probe_config == 4:
            step()
            step()
        elif args.probe_config == 1:
            ids1, mask1 = synth.config_inputs(1)
            d_i1, d_m1 = _hip.DeviceBuffer.from_array(ids1), _hip.DeviceBuffer.from_array(mask1)
            d_o1 = _hip.DeviceBuffer(D * 4)
            cps = [model] + [llmembed.Embedder.load(path).model() for _ in range(2)]
            for i in range(60):  # 30 warm-ups (graph capture), then the 30 forwards a trace reads
                check(L_.lle_embed_batch_async(cps[i % 3].h, d_i1.ptr, d_m1.ptr, 1, ids1.shape[1], D, d_o1.ptr,
                                               stream.h))
                stream.synchronize()
            log("[bench] config-1 probe: 60 forwards (the last 30 after warm-up), rotated over 3 model copies")
        else:
            ids_p, mask_p = synth.config_inputs(args.probe_config)
            mp = llmembed.Embedder.load(synth.model_path(spec, synth.CONFIG_MIX[args.probe_config],
                                                         synth.CONFIG_SEED + args.probe_config)).model()
            dip, dmp = _hip.DeviceBuffer.from_array(ids_p), _hip.DeviceBuffer.from_array(mask_p)
            dop = _hip.DeviceBuffer(ids_p.shape[0] * D * 4)
            for _ in range(2):
                check(L_.lle_embed_batch_async(mp.h, dip.ptr, dmp.ptr, ids_p.shape[0], ids_p.shape[1], D, dop.ptr,
                                               stream.h))
            stream.synchronize()
        n = 256 << 20
        src, dst = _hip.DeviceBuffer(n), _hip.DeviceBuffer(n)
        _hip._ok(_hip.rt().hipMemset(src.ptr, 1, n), "hipMemset")
        _hip._ok(_hip.rt().hipMemcpy(dst.ptr, src.ptr, n, _hip.D2D), "hipMemcpy")
        _hip.synchronize()
        nfw = 60 if args.probe_config == 1 else 2
        log(f"[bench] traffic probe done: {nfw} config-{args.probe_config} forwards, 1 copy of 268435456 B")
        return

    for _ in range(args.warmup):
        step()
    _hip.synchronize()
    # Per-kernel shares from an instrumented pass before the timed region: HIP events around
    # every launch and a synchronisation per forward (about 3% slower than plain forwards).
    share_steps = max(3, args.steps // 4)
    model.set_timing(True)
    for _ in range(share_steps):
        step()
    kt = model.timing()
    model.set_timing(False)
    dname = max(kt.items(), key=lambda kv: kv[1]["total_ms"])[0]  # dominant kernel class
    # Timed region: plain forwards, with HIP events on `stream` around the dominant kernel's
    # launches only (no per-forward synchronisation), read after the region ends.
    model.set_timing_kernel(dname)
    _hip.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    _hip.synchronize()
    t1 = time.perf_counter()
    kt_dom = model.timing()
    model.set_timing(False)
    sec = t1 - t0
    value = B * args.steps / sec
    ms_per_step = 1000.0 * sec / args.steps
    out = d_out.download((B, D), np.float32)
    norms = np.linalg.norm(out.astype(np.float64), axis=1)
    assert np.all(np.isfinite(out)) and np.abs(norms - 1).max() < 1e-3, "bench output is not L2-normalised"
    log(f"[bench] c4: {value:.1f} emb/s, {ms_per_step:.3f} ms/step")

    kernels = {k: dict(avg_ms=v["total_ms"] / max(v["launches"], 1), launches_per_step=v["launches"] / share_steps,
                       share=v["total_ms"] / max(sum(x["total_ms"] for x in kt.values()), 1e-9))
               for k, v in kt.items()}
    for k, v in sorted(kernels.items(), key=lambda kv: -kv[1]["share"]):
        log(f"[bench]   {k:12s} avg {v['avg_ms']:.4f} ms  x{v['launches_per_step']:.0f}/step  {100 * v['share']:.1f}%")
    # dominant kernel, timed live in the timed region
    dv = kt_dom[dname]
    assert dv["launches"] == kernels[dname]["launches_per_step"] * args.steps, "dominant-kernel launch count"
    avg_s = dv["total_ms"] / dv["launches"] / 1000.0
    T = B * L
    if dname.startswith("gemm"):
        K_, N_ = {"gemm_qkv": (D, 3 * D), "gemm_out_ln": (D, D), "gemm_upgate": (D, 2 * model.ffn_dim),
                  "gemm_down_ln": (model.ffn_dim, D)}[dname]
        flops = 2.0 * T * N_ * K_  # every position of config 4 is a valid token
        traffic, tsrc = committed_traffic(dname)
        roof = dict(kernel=dname, bound="mfma", achieved=flops / avg_s / 1e12, peak=PEAK_F16_TFLOPS, unit="TFLOP/s",
                    frac=flops / avg_s / 1e12 / PEAK_F16_TFLOPS, traffic=traffic, traffic_source=tsrc,
                    per_launch=f"2*M*N*K = 2*{T}*{N_}*{K_} FLOP", avg_launch_ms=avg_s * 1e3)
    else:
        roof = dict(kernel=dname, bound="hbm", achieved=dv["bytes"] / dv["launches"] / avg_s / 1e9, peak=PEAK_HBM_GBS,
                    unit="GB/s", frac=dv["bytes"] / dv["launches"] / avg_s / 1e9 / PEAK_HBM_GBS, traffic=None,
                    avg_launch_ms=avg_s * 1e3)
    total_flops = 226492416.0 * T + 4.0 * D * model.num_layers * B * L * L
    model_tflops = total_flops / (sec / args.steps) / 1e12

    # ---------------------------------------------------------------- config 1 latency
    # B=1, L=8 on the same Q8_0 model. Device time per forward from HIP events on the stream
    # (p50/p90 over --latency-iters after 20 warm-ups); "cold" rotates over three resident
    # copies of the model (3 x 120 MB of weights > the 256 MB MALL) so every forward streams
    # its weights from HBM; "warm" repeats one copy. Host-synchronised wall latency is reported
    # beside them.
    ids1, mask1 = synth.config_inputs(1)
    d_ids1, d_mask1 = _hip.DeviceBuffer.from_array(ids1), _hip.DeviceBuffer.from_array(mask1)
    d_out1 = _hip.DeviceBuffer(D * 4)
    L1 = ids1.shape[1]
    copies = [model] + ([llmembed.Embedder.load(path).model() for _ in range(2)] if args.latency_iters > 0 else [])
    ev0, ev1 = _hip.Event(), _hip.Event()

    def fwd1(mm):
        check(L_.lle_embed_batch_async(mm.h, d_ids1.ptr, d_mask1.ptr, 1, L1, D, d_out1.ptr, stream.h))

    def lat_events(models_):
        for i in range(20):
            fwd1(models_[i % len(models_)])
        stream.synchronize()
        ts = []
        for i in range(args.latency_iters):
            ev0.record(stream)
            fwd1(models_[i % len(models_)])
            ev1.record(stream)
            stream.synchronize()
            ts.append(ev0.elapsed_ms(ev1))
        return np.array(ts)

    p50 = p90 = w50 = wall50 = c1_roof = None
    if args.latency_iters > 0:  # --latency-iters 0 (profiling runs): config 4 only
        cold, warm = lat_events(copies), lat_events([model])
        wall = []
        for _ in range(args.latency_iters):
            a = time.perf_counter()
            fwd1(model)
            stream.synchronize()
            wall.append(time.perf_counter() - a)
        wall = np.array(wall) * 1e3
        v1 = d_out1.download((D,), np.float32)
        assert abs(float(np.linalg.norm(v1.astype(np.float64))) - 1) < 1e-3, "config-1 output is not L2-normalised"
        p50, p90 = float(np.percentile(cold, 50)), float(np.percentile(cold, 90))
        w50 = float(np.percentile(warm, 50))
        wall50 = float(np.percentile(wall, 50))
        c1_bytes = 120487296.0  # Q8_0 weights + gathered token rows + LN params per forward
        c1_roof = dict(bound="hbm", achieved=c1_bytes / (p50 * 1e-3) / 1e9, peak=PEAK_HBM_GBS, unit="GB/s",
                       frac=c1_bytes / (p50 * 1e-3) / 1e9 / PEAK_HBM_GBS,
                       per_forward=f"{c1_bytes:.0f} B (weights read once + token rows + LN params)")
        log(f"[bench] c1 device p50 {p50:.3f} ms p90 {p90:.3f} ms (cold MALL), warm p50 {w50:.3f} ms, "
            f"host wall p50 {wall50:.3f} ms; HBM roofline {100 * c1_roof['frac']:.2f}%")
    del copies

    # ---------------------------------------------------------------- other configs
    # Config 4 on Q6_K and Q5_K_M weights, config 3 (B=64, lengths U[16,128] padded to 128,
    # Q4_K_M) and config 5 (B=8, lengths U[1024,2048] padded to 2048, Q8_0): throughput over
    # valid sequences, per-kernel shares, and config 5's attention share and HBM rate.
    extras = {}
    if args.extras:
        def run_cfg(cfg, mix, steps):
            ids_c, mask_c = synth.config_inputs(cfg)
            Bc, Lc = ids_c.shape
            mm = llmembed.Embedder.load(synth.model_path(spec, mix, synth.CONFIG_SEED + cfg)).model()
            di, dm = _hip.DeviceBuffer.from_array(ids_c), _hip.DeviceBuffer.from_array(mask_c)
            do = _hip.DeviceBuffer(Bc * D * 4)

            def st_():
                check(L_.lle_embed_batch_async(mm.h, di.ptr, dm.ptr, Bc, Lc, D, do.ptr, stream.h))

            st_()
            _hip.synchronize()
            mm.set_timing(True)  # per-kernel shares from an instrumented pass
            for _ in range(max(2, steps // 4)):
                st_()
            kt_c = mm.timing()
            mm.set_timing(False)
            _hip.synchronize()
            t_a = time.perf_counter()
            for _ in range(steps):
                st_()
            _hip.synchronize()
            t_b = time.perf_counter()
            o_c = do.download((Bc, D), np.float32)
            assert np.all(np.isfinite(o_c)), f"config {cfg} {mix}: non-finite output"
            # the same sequences back to back on the device (lle_embed_packed_async)
            lens_c = mask_c.sum(axis=1).astype(np.int64)
            packed_c = np.concatenate([ids_c[b, :lens_c[b]] for b in range(Bc)]).astype(np.int32)
            off_c = np.concatenate([[0], np.cumsum(lens_c)]).astype(np.int32)
            dpi, dpo, dpy = (_hip.DeviceBuffer.from_array(packed_c), _hip.DeviceBuffer.from_array(off_c),
                             _hip.DeviceBuffer(Bc * D * 4))

            def stp():
                check(L_.lle_embed_packed_async(mm.h, dpi.ptr, dpo.ptr, Bc, int(packed_c.size), Lc, D, dpy.ptr,
                                                stream.h))

            stp()
            _hip.synchronize()
            assert np.array_equal(dpy.download((Bc, D), np.float32).view(np.uint32), o_c.view(np.uint32)), \
                f"config {cfg}: packed device entry != padded"
            t_p = time.perf_counter()
            for _ in range(steps):
                stp()
            _hip.synchronize()
            packed_s = (time.perf_counter() - t_p) / steps
            # host-pointer entry point: padding is packed away before the first kernel
            emb_c = llmembed.Embedder(mm)
            h_c = emb_c.embed_padded(ids_c, mask_c)
            assert np.array_equal(h_c.view(np.uint32), o_c.view(np.uint32)), f"config {cfg}: packed != padded"
            t_c = time.perf_counter()
            for _ in range(steps):
                emb_c.embed_padded(ids_c, mask_c)
            host_s = (time.perf_counter() - t_c) / steps
            tot_ms = sum(v["total_ms"] for v in kt_c.values())
            ms = 1000.0 * (t_b - t_a) / steps
            r = dict(mix=mix, batch=int(Bc), seq_len=int(Lc), valid_tokens=int(mask_c.sum()),
                     emb_per_s=Bc * steps / (t_b - t_a), ms_per_step=ms,
                     device_packed_emb_per_s=Bc / packed_s, device_packed_ms=1e3 * packed_s,
                     host_api_packed_emb_per_s=Bc / host_s, host_api_packed_ms=1e3 * host_s,
                     shares={k: round(v["total_ms"] / tot_ms, 4) for k, v in kt_c.items()})
            if "attention" in kt_c:
                at = kt_c["attention"]
                r["attention_share"] = at["total_ms"] / tot_ms
                r["attention_algorithmic_gbs"] = at["bytes"] / (at["total_ms"] * 1e-3) / 1e9
            log(f"[bench] config {cfg} {mix}: {r['emb_per_s']:.1f} emb/s, {ms:.3f} ms/step; packed on device "
                f"{Bc / packed_s:.1f} emb/s; host API (packed rows) {Bc / host_s:.1f} emb/s"
                + (f", attention {100 * r['attention_share']:.1f}% of kernel time at {r['attention_algorithmic_gbs']:.0f} GB/s (Q,K,V,O bytes)"
                   if "attention_share" in r else ""))
            mm.close()
            return r

        extras["config4_Q6_K"] = run_cfg(4, "Q6_K", 5)
        extras["config4_Q5_K_M"] = run_cfg(4, "Q5_K_M", 5)
        extras["config3_Q4_K_M"] = run_cfg(3, "Q4_K_M", 10)
        extras["config5_Q8_0"] = run_cfg(5, "Q8_0", 5)

        # Config 2: the isolated quantised projections Y = X W^T at the encoder's four shapes,
        # M in {8, 512, 32768}, four formats; X f16 resident on the device (lle_gemm_f16_async),
        # device time per call from HIP events (median of 20); for M = 8 also a back-to-back
        # sequence over distinct weight copies (HBM streaming). Roofline: the dense fp16 MFMA peak
        # for FLOP/s, and for bytes the quantised W + X f16 + Y f32 read/written once. For
        # M >= 512 also the call as config 2 states it, on f32 X in HBM (lle_gemm_async: the
        # f32 -> f16 pass, then the GEMM), with bytes W + X f32 + Y f32.
        from llmembed import quant as q_

        c2 = []
        rng2 = np.random.default_rng(0xC2)
        xbuf = _hip.DeviceBuffer(32768 * 3072 * 2)
        ybuf = _hip.DeviceBuffer(32768 * 3072 * 4)
        pbuf = _hip.DeviceBuffer(4 * 1024 * 3072 * 4)  # split-K partials below 1024 rows
        xbuf_h = rng2.standard_normal(32768 * 3072, dtype=np.float32)
        xbuf.upload(xbuf_h.astype(np.float16))
        x32buf = _hip.DeviceBuffer.from_array(xbuf_h)  # config 2's f32 X
        del xbuf_h
        e0, e1 = _hip.Event(), _hip.Event()
        for tname, t in (("Q8_0", q_.Q8_0), ("Q6_K", q_.Q6_K), ("Q5_K", q_.Q5_K), ("Q4_K", q_.Q4_K)):
            for K_c, N_c in ((768, 2304), (768, 768), (768, 3072), (3072, 768)):
                wq = q_.quantize(t, (rng2.standard_normal((N_c, K_c)) * 0.02).astype(np.float32), rng2)
                W = llmembed.Weight(t, wq, K_c, N_c)
                for M_c in (8, 512, 32768):
                    def call():
                        W.gemm_f16_async(xbuf.value, M_c, ybuf.value, pbuf.value if M_c < 1024 else 0, stream.h.value)
                    for _ in range(3):
                        call()
                    ts = []
                    for _ in range(20):
                        e0.record(stream)
                        call()
                        e1.record(stream)
                        ts.append(e0.elapsed_ms(e1))
                    ms = float(np.median(ts))
                    flops = 2.0 * M_c * N_c * K_c
                    nbytes = float(wq.nbytes) + M_c * K_c * 2 + M_c * N_c * 4
                    r2 = dict(fmt=tname, K=K_c, N=N_c, M=M_c, us=1e3 * ms, tflops=flops / ms / 1e9,
                              mfma_frac=flops / ms / 1e9 / PEAK_F16_TFLOPS, gbs=nbytes / ms / 1e6,
                              hbm_frac=nbytes / ms / 1e6 / PEAK_HBM_GBS)
                    if M_c >= 512:  # f32 X as config 2 states it
                        def call32():
                            W.gemm_async(x32buf.value, xbuf.value, M_c, ybuf.value, stream.h.value)
                        call32()
                        ts = []
                        for _ in range(20):
                            e0.record(stream)
                            call32()
                            e1.record(stream)
                            ts.append(e0.elapsed_ms(e1))
                        ms32 = float(np.median(ts))
                        b32 = float(wq.nbytes) + M_c * K_c * 4 + M_c * N_c * 4
                        r2.update(us_f32x=1e3 * ms32, tflops_f32x=flops / ms32 / 1e9, gbs_f32x=b32 / ms32 / 1e6)
                    if M_c == 8:
                        # weight streaming from HBM: back-to-back calls over distinct copies of the
                        # weight (>= 520 MB in all, past the 256 MB MALL), device time of the sequence
                        n_cp = min(2048, -(-520 * 2 ** 20 // wq.nbytes))
                        os.environ["LLE_NO_F16_COPY"] = "1"  # M = 8 streams the quantised planes only
                        try:
                            cps = [llmembed.Weight(t, wq, K_c, N_c) for _ in range(n_cp)]
                        finally:
                            del os.environ["LLE_NO_F16_COPY"]
                        for Wc in cps[:64]:
                            Wc.gemm_f16_async(xbuf.value, 8, ybuf.value, pbuf.value, stream.h.value)
                        e0.record(stream)
                        for Wc in cps:
                            Wc.gemm_f16_async(xbuf.value, 8, ybuf.value, pbuf.value, stream.h.value)
                        e1.record(stream)
                        ms_seq = e0.elapsed_ms(e1) / n_cp
                        for Wc in cps:
                            Wc.close()
                        r2.update(seq_copies=n_cp, seq_us=1e3 * ms_seq, seq_gbs=nbytes / ms_seq / 1e6,
                                  seq_hbm_frac=nbytes / ms_seq / 1e6 / PEAK_HBM_GBS)
                    c2.append(r2)
                W.close()
        extras["config2"] = c2
        for r in c2:
            if r["fmt"] in ("Q8_0", "Q4_K"):
                log(f"[bench] config 2 {r['fmt']:4s} K={r['K']:4d} N={r['N']:4d} M={r['M']:5d}: {r['us']:8.1f} us "
                    f"{r['tflops']:7.1f} TFLOP/s ({100 * r['mfma_frac']:4.1f}% MFMA) {r['gbs']:7.0f} GB/s "
                    f"({100 * r['hbm_frac']:4.1f}% HBM)"
                    + (f"; back-to-back over {r['seq_copies']} weight copies {r['seq_us']:.2f} us "
                       f"{r['seq_gbs']:.0f} GB/s ({100 * r['seq_hbm_frac']:.1f}% HBM)" if "seq_us" in r else ""))
        del xbuf, ybuf, pbuf, x32buf

        # LLE_PRECISION_F32 (the reference's own f32 arithmetic): config 4 through the host entry
        # (embeddings compared with the CPU oracle's bit for bit below) and config 1's latency
        model.set_precision("f32")
        emb.embed_padded(ids[:2], mask[:2])
        _hip.synchronize()
        a = time.perf_counter()
        out32 = emb.embed_padded(ids, mask)
        f32_c4_s = time.perf_counter() - a
        emb.embed(ids1[0], mask1[0])
        ts = []
        for _ in range(30):
            a = time.perf_counter()
            emb.embed(ids1[0], mask1[0])
            ts.append(time.perf_counter() - a)
        model.set_precision("f16")
        extras["precision_f32"] = dict(c4_emb_per_s=B / f32_c4_s, c4_ms=1e3 * f32_c4_s,
                                       c1_host_wall_p50_ms=1e3 * float(np.percentile(ts, 50)),
                                       note="host entries (PCIe included); config-4 rows compared with the CPU "
                                            "oracle bit for bit in cpu_baseline")
        log(f"[bench] F32 precision: config 4 {B / f32_c4_s:.0f} emb/s ({1e3 * f32_c4_s:.1f} ms), config 1 "
            f"{1e3 * float(np.percentile(ts, 50)):.2f} ms (host wall p50)")

        # Text path (EmbedBatch over strings): native host tokeniser, then lle_embed_texts'
        # length-ordered batches, against the same texts in input order, 256 per padded batch.
        corpus = synth.texts(4096, seed=0x7E57, min_words=4, max_words=110)
        nbytes = sum(len(t.encode()) for t in corpus)
        tk = emb.tokenizer
        tk.encode_batch(corpus[:256], model.max_seq_len, prefix=emb.task_prefix)
        a = time.perf_counter()
        _, _, cnt = tk.encode_batch(corpus, model.max_seq_len, prefix=emb.task_prefix)
        tok_s = time.perf_counter() - a
        emb.embed_texts(corpus[:512])
        a = time.perf_counter()
        vec = emb.embed_texts(corpus)
        e2e_s = time.perf_counter() - a
        a = time.perf_counter()
        padded_tokens = 0
        naive = []
        for i in range(0, len(corpus), 256):
            ib, mb, _ = tk.encode_batch(corpus[i:i + 256], model.max_seq_len, prefix=emb.task_prefix)
            padded_tokens += ib.size
            naive.append(emb.embed_padded(ib, mb))
        naive_s = time.perf_counter() - a
        naive = np.concatenate(naive)
        assert np.array_equal(naive.view(np.uint32), vec.view(np.uint32)), "text path: batching changed a row"
        extras["texts"] = dict(
            texts=len(corpus), bytes=nbytes, tokens=int(cnt.sum()), mean_tokens=float(cnt.mean()),
            tokenize_ms=1e3 * tok_s, tokenize_mb_per_s=nbytes / tok_s / 1e6, tokenize_tokens_per_s=cnt.sum() / tok_s,
            e2e_texts_per_s=len(corpus) / e2e_s, e2e_valid_tokens_per_s=cnt.sum() / e2e_s,
            input_order_texts_per_s=len(corpus) / naive_s,
            input_order_padding_fraction=1 - cnt.sum() / padded_tokens,
            note="synthetic texts (synth.texts) over the synthetic 30522-token vocabulary, config-4 model; e2e = "
                 "tokenise + ordered batches + GPU + copies; input order = 256-text padded batches, same rows bit for bit")
        log(f"[bench] texts: tokenise {nbytes / tok_s / 1e6:.1f} MB/s ({cnt.sum() / tok_s / 1e6:.2f} M tok/s); "
            f"embed_texts {len(corpus) / e2e_s:.0f} texts/s vs {len(corpus) / naive_s:.0f} in input order "
            f"({100 * extras['texts']['input_order_padding_fraction']:.0f}% padding)")

    # ---------------------------------------------------------------- CPU baseline
    cpu = None
    if args.cpu_seqs > 0:
        import oracle

        om = oracle.OracleModel(path)
        S = min(args.cpu_seqs, B)
        om.embed_batch(ids[:1], mask[:1])  # warm-up (page in the dequantised weights)
        a = time.perf_counter()
        ref = om.embed_batch(ids[:S], mask[:S])
        cs = time.perf_counter() - a
        try:
            ncores = len(os.sched_getaffinity(0))
        except AttributeError:  # pragma: no cover
            ncores = os.cpu_count()
        workers = min(os.cpu_count() or 1, S, 8)
        cos = np.sum(ref * out[:S], axis=1) / np.linalg.norm(ref, axis=1) / np.linalg.norm(out[:S], axis=1)
        max_abs = float(np.abs(ref.astype(np.float64) - out[:S]).max())
        cpu = dict(value=S / cs, unit="embeddings/s", cores=min(ncores, workers * min(os.cpu_count() or 1, 8)),
                   kind="port",
                   sample=(f"C oracle (restatement of the reference pure-Go AVX-512 GemmPrePacked32 path) on the first "
                           f"{S} of the {B} config-4 sequences (L={L}), {workers} EmbedBatch workers x "
                           f"{min(os.cpu_count() or 1, 8)} GEMM threads, {cs:.1f} s wall on {ncores} available cores"),
                   gpu_vs_cpu_min_cos=float(cos.min()), gpu_vs_cpu_max_abs=max_abs)
        log(f"[bench] cpu oracle {S / cs:.2f} emb/s ({cs:.1f} s); vs GPU over {S} rows: min cos {cos.min():.7f}, "
            f"max abs {max_abs:.2e}")
        if "precision_f32" in extras:
            eq = int(np.all(out32[:S].view(np.uint32) == ref.view(np.uint32), axis=1).sum())
            extras["precision_f32"]["c4_rows_bit_equal_to_cpu"] = f"{eq}/{S}"
            cpu["f32_precision_rows_bit_equal"] = f"{eq}/{S}"
            log(f"[bench] F32 precision rows bit-equal to the CPU oracle: {eq}/{S}")
        assert cos.min() >= 0.9999 and max_abs <= 1e-3, "GPU rows outside the parity bar against the oracle"
        # host CPU identity, and config 1 on the CPU: p50 wall time of one L=8 sequence over 50 runs
        model_name, avx512 = None, None
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name") and model_name is None:
                        model_name = line.split(":", 1)[1].strip()
                    elif line.startswith("flags") and avx512 is None:
                        avx512 = "avx512f" in line.split()
        except OSError:
            pass
        cpu.update(cpu_model=model_name, avx512f=avx512, nproc=os.cpu_count(), affinity_cores=ncores)
        if args.latency_iters > 0:
            om.embed(ids1[0], mask1[0])
            ts = []
            for _ in range(50):
                a = time.perf_counter()
                v1c = om.embed(ids1[0], mask1[0])
                ts.append(time.perf_counter() - a)
            cpu["c1_p50_ms"] = 1e3 * float(np.percentile(ts, 50))
            cpu["c1_sample"] = (f"config 1 (B=1, L={L1}) through the same C oracle, {min(os.cpu_count() or 1, 8)} "
                                "GEMM threads, p50 wall over 50 runs after one warm-up")
            log(f"[bench] cpu oracle c1 p50 {cpu['c1_p50_ms']:.2f} ms; cos vs GPU "
                f"{float(np.dot(v1c, v1) / np.linalg.norm(v1c) / np.linalg.norm(v1)):.7f}")

    res = {
        "metric": "embeddings/sec at B=256,L=128 Q8_0",
        "value": value,
        "unit": "embeddings/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": f"config 4: full 12-layer nomic-bert (d=768, 12 heads, FFN 3072), random-init "
                               f"N(0,0.02) {args.mix} GGUF, B={B}, L={L}, all positions valid",
                   "batch": B, "seq_len": L, "quant": args.mix},
        "model_tflops": model_tflops,
        "p50_ms_b1_l8": p50,
        "p90_ms_b1_l8": p90,
        "p50_ms_b1_l8_warm_mall": w50,
        "p50_ms_b1_l8_host_wall": wall50,
        "roofline_b1_l8": c1_roof,
        "kernels": kernels,
        "roofline": roof,
        "cpu_baseline": cpu,
        "gpu_vs_cpu": (value / cpu["value"]) if cpu else None,
        "other_configs": extras,
    }
    print(json.dumps(res), flush=True)



if __name__ == "__main__":
    main()
