#!/usr/bin/env python3
"""Benchmark of the chromoFold decode-in-kernel hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload kv|rrr]

Prints ONE JSON line (the driver's contract). The headline workload is BASELINE.json configs[3]: compressed
paged-KV attention decode at Llama-3-8B layer shape (32 q heads, 8 KV heads, head_dim 128, 16-token pages,
int8 per-page-per-head absmax scale + rANS per page), context 32768, batch 32. One step = one decode token for all
32 sequences through one layer. The wavelet-rank figure (configs[0] shape, 1M rank queries) rides along under
"secondary". Inputs are seeded synthetic data already resident in HBM when timing starts.

Timing: untimed back-to-back launches for at least 3 s (and at least W of them), so that the chip's clocks settle
where they stay under continuous load, then exactly K steps bracketed by torch.cuda.synchronize(); per-launch kernel
durations come from HIP events recorded on the stream the kernels run on (torch's current stream, whose handle
is what the C ABI receives).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the dominant kernel, from rocprofv3 FETCH_SIZE + WRITE_SIZE runs calibrated on a copy of
# known size (profiles/kv_batched_c4_32k.md): only quoted for the workload shape it was measured on.
# For the FM search kernels the index is cache-resident, so FETCH_SIZE there is the L2-miss traffic that the
# Infinity Cache (or HBM) serves (profiles/fm_c2.md).
MEASURED_TRAFFIC = {("kv", 32768, 32): 2.0848e9, ("fm_count", 1 << 24, 1_000_000): 95.537e9,
                    ("fm_locate", 1 << 24, 900_000): 49.336e9, ("fm_count_lines", 1 << 24, 1_000_000): 32.44e9,
                    ("fm_locate_lines", 1 << 24, 900_000): 25.99e9, ("fm_count_quads", 1 << 24, 1_000_000): 18.82e9,
                    ("fm_locate_quads", 1 << 24, 900_000): 14.84e9}
METRIC = "compressed-KV attn decode tokens/s + HBM GB/s fraction; wavelet rank Mq/s"


def _events_time(fn, steps: int, warmup: int, warm_s: float = 0.05):
    """Run fn() back to back for at least `warmup` launches and warm_s seconds (clocks at their sustained state),
    then `steps` times each bracketed by events; returns (total_ms_wall, per_launch_ms)."""
    import torch
    if warmup > 0 or warm_s > 0:
        _warm(fn, warmup, warm_s)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    per = [a.elapsed_time(b) for a, b in evs]
    return wall_ms, per


def bench_copy(steps: int, warmup: int, nbytes: int = 1 << 30) -> dict:
    """Device-to-device copy of `nbytes` (torch's copy kernel): the measured stream-copy peak the HBM fractions are
    also quoted against, and the known-size kernel that FETCH_SIZE / WRITE_SIZE counters are calibrated on."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda:0")
    dst = torch.empty_like(src)
    _, per = _events_time(lambda: dst.copy_(src), steps, warmup)
    t = float(np.median(per)) * 1e-3
    return {"copy_bytes": nbytes, "copy_ms": t * 1e3, "stream_copy_gbs": 2.0 * nbytes / t / 1e9}


# ------------------------------------------------------------------------------------------------ RRR wavelet (C1)
def bench_rrr(steps: int, warmup: int, cpu: bool = True) -> dict:
    import torch
    from chromofold_amd import synth
    from chromofold_amd.search import build_rrrw, to_u32, u32_dev

    n, vocab, nq = 1 << 20, 32000, 1 << 20
    tok = synth.zipf_tokens(n, vocab, 1.1, synth.SEED_C1)
    dtok = torch.from_numpy(tok.view(np.int32)).to("cuda:0")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    idx, lay = build_rrrw(dtok, 15)  # on-device index construction (cf_rrrw_build)
    t_build = time.perf_counter() - t0
    pos, c, i = synth.rrr_queries(tok, nq, vocab, synth.SEED_C1 + 1)
    dpos, dc, di = u32_dev(pos), u32_dev(c), u32_dev(i)
    out = torch.empty(nq, dtype=torch.int32, device="cuda:0")
    # correctness gate before timing: access against the token array itself (closed form)
    idx.access_into(dpos, out)
    assert np.array_equal(to_u32(out), tok[pos]), "access mismatch"
    idx.rank_into(dc, di, out)
    rank_gpu = to_u32(out)

    # the derived line layout (built once at load): same results, timed beside the RRR kernels
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    idx.build_lines()
    torch.cuda.synchronize()
    t_lines = time.perf_counter() - t0
    out_l = torch.empty_like(out)
    idx.rank_lines_into(dc, di, out_l)
    assert np.array_equal(to_u32(out_l), rank_gpu), "line-layout rank != RRR rank"
    idx.access_lines_into(dpos, out_l)
    assert np.array_equal(to_u32(out_l), tok[pos]), "line-layout access mismatch"

    # the derived 4-ary layout (built once at load): 8 records per query instead of 15; the C1 figures
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    idx.build_quads(n)
    torch.cuda.synchronize()
    t_quads = time.perf_counter() - t0
    idx.rank_quads_into(dc, di, out_l)
    assert np.array_equal(to_u32(out_l), rank_gpu), "4-ary layout rank != RRR rank"
    idx.access_quads_into(dpos, out_l)
    assert np.array_equal(to_u32(out_l), tok[pos]), "4-ary layout access mismatch"
    wall_r, per_r = _events_time(lambda: idx.rank_quads_into(dc, di, out_l), steps, warmup)
    _, per_a = _events_time(lambda: idx.access_quads_into(dpos, out_l), steps, warmup)
    _, per_lr = _events_time(lambda: idx.rank_lines_into(dc, di, out_l), steps, warmup)
    _, per_la = _events_time(lambda: idx.access_lines_into(dpos, out_l), steps, warmup)
    _, per_rr = _events_time(lambda: idx.rank_into(dc, di, out), steps, warmup)
    _, per_ra = _events_time(lambda: idx.access_into(dpos, out), steps, warmup)
    t_rank, t_acc, t_lrank, t_lacc, t_rrank, t_racc = (float(np.mean(x)) * 1e-3 for x in
                                                       (per_r, per_a, per_lr, per_la, per_rr, per_ra))
    # algorithmic bytes: 4-ary layout = 8 levels x one 64-B record per query (rank and access alike) + the query
    # words + the result; line layout = 15 levels x 64 B; RRR = 15 levels x 32 B per rank1 (samples 12 + class scan
    # 16 + offset 4), 2 rank1 per level for rank (960 B), 1 for access (480 B)
    L4 = (15 + 1) // 2
    bytes_rank = nq * (L4 * 64 + 12.0)
    bytes_acc = nq * (L4 * 64 + 8.0)
    res = {
        "rank_mqs": nq / t_rank / 1e6, "access_mqs": nq / t_acc / 1e6,
        "rank_ms": t_rank * 1e3, "access_ms": t_acc * 1e3,
        "rank_wall_ms_per_step": wall_r / steps,
        "rank_roofline": {"bound": "hbm (nominal; the index is L2-resident)", "achieved": bytes_rank / t_rank / 1e9,
                          "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": bytes_rank / t_rank / 1e9 / HBM_PEAK_GBS,
                          "traffic": None},
        "access_gbs": bytes_acc / t_acc / 1e9,
        "lines_rank_mqs": nq / t_lrank / 1e6, "lines_access_mqs": nq / t_lacc / 1e6,
        "lines_rank_ms": t_lrank * 1e3, "lines_access_ms": t_lacc * 1e3,
        "quads_bytes": idx.quads.numel(), "quads_build_ms": t_quads * 1e3,
        "rrr_rank_mqs": nq / t_rrank / 1e6, "rrr_access_mqs": nq / t_racc / 1e6,
        "rrr_rank_ms": t_rrank * 1e3, "rrr_access_ms": t_racc * 1e3,
        "rrr_rank_gbs": 960.0 * nq / t_rrank / 1e9,
        "index_bytes": idx.device_bytes(), "bits_per_token": idx.device_bytes() * 8.0 / n,
        "lines_bytes": idx.lines.numel(), "lines_build_ms": t_lines * 1e3,
        "gpu_index_build_ms": t_build * 1e3,
    }
    if cpu:
        import oracle as O
        w = O.rrrw_build(tok, 15)  # the CPU baseline's own index (byte-identical to the GPU build)
        th = O.num_threads()
        t0 = time.perf_counter()
        ref = O.rrrw_rank(w, c, i)
        dt = time.perf_counter() - t0
        assert np.array_equal(ref, rank_gpu), "GPU rank != oracle rank"
        res["cpu_baseline"] = {"value": nq / dt / 1e6, "unit": "Mq/s", "cores": th, "kind": "port",
                               "sample": f"1M rank queries on the C1 index (oracle, OpenMP {th} threads)"}
    return res


# ------------------------------------------------------------------------------------------------ FM-index (C2)
def bench_fm(steps: int, warmup: int, cpu: bool = True) -> dict:
    """16M Zipf tokens, vocab 32000: GPU suffix array + BWT + RRR wavelet build, then count of 1M patterns (900K cut
    from the text, 100K random) and locate of every occurrence of the cut patterns."""
    import torch
    from chromofold_amd import synth
    from chromofold_amd.search import build_fm

    n, vocab = 1 << 24, 32000
    tok = synth.zipf_tokens(n, vocab, 1.1, synth.SEED_C2)
    dtok = torch.from_numpy(tok.view(np.int32)).to("cuda:0")
    fm, info = build_fm(dtok, 32)
    flat, pstart, plen = synth.fm_patterns(tok, 900_000, 100_000, vocab, synth.SEED_C2 + 1)
    dpat, dps, dpl = (torch.from_numpy(a).to("cuda:0") for a in (flat, pstart, plen))
    cnt = fm.count(dpat, dps, dpl)
    lo, hi = fm.ranges(dpat, dps, dpl)
    occ = int((hi - lo).sum().item())
    # every occurrence row of every pattern, flattened on the device
    rows = (torch.repeat_interleave(lo, (hi - lo).long()) +
            torch.arange(occ, device="cuda:0", dtype=torch.int32) -
            torch.repeat_interleave(torch.cumsum(hi - lo, 0, dtype=torch.int32) - (hi - lo), (hi - lo).long()))
    rows = rows.to(torch.int32).contiguous()
    pos = torch.empty_like(rows)
    fm.locate(rows, pos)
    torch.cuda.synchronize()
    # gate (size-independent): cut patterns occur, counts agree with ranges, every located position spells its
    # pattern in the text
    c_h = cnt.cpu().numpy()
    assert (c_h[:900_000] >= 1).all() and np.array_equal(c_h, (hi - lo).cpu().numpy())
    s = np.concatenate([tok.astype(np.int64) + 1, [0]])
    rng = np.random.default_rng(5)
    owner = np.repeat(np.arange(c_h.size), c_h)
    p_h = pos.cpu().numpy()
    for k in rng.integers(0, occ, 2000):
        j = owner[k]
        a = int(p_h[k])
        assert np.array_equal(s[a:a + plen[j]], flat[pstart[j]:pstart[j] + plen[j]]), "located position mismatch"
    # the derived line layout (built once at load): same results, timed beside the RRR kernels
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fm.build_lines()
    torch.cuda.synchronize()
    t_lines_build = time.perf_counter() - t0
    cnt_l = fm.count_lines(dpat, dps, dpl)
    lo_l, hi_l = fm.ranges_lines(dpat, dps, dpl)
    pos_l = torch.empty_like(rows)
    fm.locate_lines(rows, pos_l)
    assert torch.equal(cnt_l, cnt) and torch.equal(lo_l, lo) and torch.equal(hi_l, hi), "line layout != RRR search"
    assert torch.equal(pos_l, pos), "line layout != RRR locate"
    # the derived 4-ary layout (built once at load): 8 records per walk instead of 15; the C2 figures
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fm.build_quads()
    torch.cuda.synchronize()
    t_quads_build = time.perf_counter() - t0
    cnt_q = fm.count_quads(dpat, dps, dpl)
    lo_q, hi_q = fm.ranges_quads(dpat, dps, dpl)
    pos_q = torch.empty_like(rows)
    fm.locate_quads(rows, pos_q)
    assert torch.equal(cnt_q, cnt) and torch.equal(lo_q, lo) and torch.equal(hi_q, hi), "4-ary layout != RRR search"
    assert torch.equal(pos_q, pos), "4-ary layout != RRR locate"
    _, per_c = _events_time(lambda: fm.count(dpat, dps, dpl), steps, warmup)
    _, per_l = _events_time(lambda: fm.locate(rows, pos), steps, warmup)
    _, per_cl = _events_time(lambda: fm.count_lines(dpat, dps, dpl, out=cnt_l), steps, warmup)
    _, per_ll = _events_time(lambda: fm.locate_lines(rows, pos_l), steps, warmup)
    _, per_cq = _events_time(lambda: fm.count_quads(dpat, dps, dpl, out=cnt_q), steps, warmup)
    _, per_lq = _events_time(lambda: fm.locate_quads(rows, pos_q), steps, warmup)
    t_c, t_l, t_cl, t_ll, t_cq, t_lq = (float(np.mean(x)) * 1e-3 for x in (per_c, per_l, per_cl, per_ll, per_cq,
                                                                          per_lq))
    res = {"count_mpats": pstart.size / t_cq / 1e6, "count_ms": t_cq * 1e3, "occurrences": occ,
           "locate_mocc": occ / t_lq / 1e6, "locate_ms": t_lq * 1e3,
           "lines_count_mpats": pstart.size / t_cl / 1e6, "lines_count_ms": t_cl * 1e3,
           "lines_locate_mocc": occ / t_ll / 1e6, "lines_locate_ms": t_ll * 1e3,
           "rrr_count_mpats": pstart.size / t_c / 1e6, "rrr_count_ms": t_c * 1e3,
           "rrr_locate_mocc": occ / t_l / 1e6, "rrr_locate_ms": t_l * 1e3,
           "gpu_sa_build_s": info["sa_s"], "gpu_index_build_s": info["build_s"], "lines_build_s": t_lines_build,
           "quads_build_s": t_quads_build, "index_bytes": fm.w.device_bytes(), "lines_bytes": fm.lines.numel(),
           "quads_bytes": fm.quads.numel()}
    # cost models (algorithmic bytes), symbols = pattern symbols per launch:
    #   RRR count: 1928 B per symbol (rank(c, lo) and rank(c, hi), each 2 rank1 per level x 15 levels x 32 B, + 8 B
    #   of C[]); RRR locate: 15.5 expected LF steps x (access 480 + rank 960 + mark word 4) + sval 4 + msb 4;
    #   line count: 1928 B per symbol (2 rank1 per level x 15 levels x one 64-B record, + lfb 4 B + the symbol 4 B);
    #   line locate: 15.5 LF steps x (15 records x 64 B + lfb 4 + mark word 4) + sval 4 + msb 4;
    #   4-ary count: 1032 B per symbol (2 walks x 8 levels x one 64-B record + lfb 4 + the symbol 4); 4-ary locate:
    #   15.5 LF steps x (8 records x 64 B + lfb 4 + mark word 4) + sval 4 + msb 4.
    syms = float(plen.astype(np.int64).sum())
    L4 = (fm.w.bits + 1) // 2
    models = {"count_roofline": (syms * (2 * L4 * 64 + 8), t_cq, ("fm_count_quads", n, pstart.size)),
              "locate_roofline": (occ * (15.5 * (L4 * 64 + 8) + 8), t_lq, ("fm_locate_quads", n, occ)),
              "lines_count_roofline": (syms * (2 * 15 * 64 + 8), t_cl, ("fm_count_lines", n, pstart.size)),
              "lines_locate_roofline": (occ * (15.5 * (15 * 64 + 8) + 8), t_ll, ("fm_locate_lines", n, occ)),
              "rrr_count_roofline": (syms * (1920 + 8), t_c, ("fm_count", n, pstart.size)),
              "rrr_locate_roofline": (occ * (15.5 * (480 + 960 + 4) + 8), t_l, ("fm_locate", n, occ))}
    for key, (b, t, tk) in models.items():
        tr = MEASURED_TRAFFIC.get(tk)
        res[key] = {"bound": "hbm (nominal; the index is cache-resident)", "achieved": b / t / 1e9,
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": b / t / 1e9 / HBM_PEAK_GBS, "model_bytes": b,
                    "traffic": tr, "traffic_gbs": tr / t / 1e9 if tr else None,
                    "traffic_over_model": tr / b if tr else None}
    if cpu:
        import oracle as O
        from chromofold_amd.search import to_u32
        w = O.RrrwArrays(fm.w.bits, fm.w.cwords, fm.w.nsb, fm.w.na,
                         *[fm.w.tensors[k].cpu().numpy().view(dt) for k, dt in
                           (("classes", np.uint32), ("offsets", np.uint32), ("rank_a", np.int32),
                            ("rank_d", np.uint16), ("off_a", np.int32), ("off_d", np.uint16),
                            ("offbase", np.int32), ("zeros", np.int32))])
        f = O.FmArrays(w, fm.tensors["C"].cpu().numpy(), to_u32(fm.tensors["mwords"]), fm.tensors["msb"].cpu().numpy(),
                       fm.tensors["sval"].cpu().numpy(), fm.sigma, fm.n, fm.sa_sample)
        k = 100_000
        th = O.num_threads()
        t0 = time.perf_counter()
        ref = O.fm_count(f, flat, pstart[:k], plen[:k])
        dt = time.perf_counter() - t0
        assert np.array_equal(ref, c_h[:k]), "GPU count != oracle count"
        res["cpu_baseline"] = {"value": k / dt / 1e6, "unit": "M patterns/s", "cores": th, "kind": "port",
                               "sample": f"count of the first {k} patterns on the same index (oracle, OpenMP {th} "
                                         f"threads)"}
    return res


# ------------------------------------------------------------------------------------------------ matmul (C3)
def bench_qw(steps: int, warmup: int, batches=(1, 4, 16, 64), codecs=("huffman", "rans")) -> dict:
    """4096 x 4096 int4 weights (N(0,1), per (row, 64-col) absmax), per-band Huffman or pair-rANS tables, bf16 x:
    y = x W^T. Roofline per batch: bytes = coded matrix + x + y over the per-call time (HBM-bound at small B)."""
    import ctypes as C
    import torch
    import oracle as O
    from chromofold_amd import _abi as A
    from chromofold_amd import qw, synth

    M = K = 4096
    REPS = 20
    rng = np.random.default_rng(synth.SEED_C3)
    W = rng.standard_normal((M, K), dtype=np.float32)
    sym, sc = qw.quantize_int4(W)
    scales = np.repeat(sc, 64, axis=1)
    xs = {B: torch.from_numpy(rng.standard_normal((B, K), dtype=np.float32)).to(torch.bfloat16) for B in batches}
    refs = {B: O.qmatmul_f64(xs[B].float().numpy(), sym, scales, 8) for B in batches if B <= 16}
    res = {}
    for name in codecs:
        codec = qw.QW_CODEC_HUFFMAN if name == "huffman" else qw.QW_CODEC_RANS
        h = qw.encode_symbols(sym, sc, codec)
        mat = qw.QwMatrix(h, "cuda:0")
        r = {"coded_bytes": h.nbytes, "bits_per_weight": h.nbytes * 8.0 / (M * K)}
        for B in batches:
            dx = xs[B].to("cuda:0")
            y = torch.empty((B, M), device="cuda:0")
            mat.matmul_into(dx, y)
            torch.cuda.synchronize()
            if B in refs:  # gate against the fp64 oracle
                err = float(np.abs(y.cpu().numpy() - refs[B]).max() / np.abs(refs[B]).max())
                assert err <= 1e-3, (name, B, err)
            # One call takes a few us, about what Python needs to issue it, so per-call events would time the host.
            # Instead REPS back-to-back calls are captured in a graph (as a model's forward pass would issue them)
            # and `steps` replays run back to back between one pair of events, the start event queued behind a
            # first replay so that the device never waits for the host to submit the next one (events around each
            # replay would add the submission gap, ~1 us per call at 20 calls a replay); every replay must
            # reproduce the eager result bit for bit.
            y_eager = y.clone()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(REPS):
                    mat.matmul_into(dx, y)
            torch.cuda.synchronize()
            _warm(g.replay, warmup, 0.1)  # sustained clocks: ~0.1 s of back-to-back calls first
            g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            assert torch.equal(y, y_eager), "graph replay differs from the eager call"
            t_graph = e0.elapsed_time(e1) * 1e-3 / (steps * REPS)
            # The same calls as plain stream launches (the C entry point called directly, its arguments prepared
            # once), steps * REPS of them between one pair of events. A graph's kernel nodes measured ~0.7 us
            # slower each than stream launches of the same kernel. The stream figure counts only when the host
            # issues the calls faster than the device runs them (host_us below us_stream, checked here).
            fn = A.lib().cf_qw_matmul_async
            args = (C.byref(mat.desc), dx.data_ptr(), y.data_ptr(), B, torch.cuda.current_stream().cuda_stream)
            bad = 0

            def stream_calls():
                nonlocal bad
                for _ in range(REPS):
                    bad |= fn(*args)

            _warm(stream_calls, warmup, 0.1)
            n = steps * REPS
            bad |= fn(*args)
            e0.record()
            h0 = time.perf_counter()
            for _ in range(n):
                bad |= fn(*args)
            host = (time.perf_counter() - h0) / n
            e1.record()
            torch.cuda.synchronize()
            assert bad == 0 and torch.equal(y, y_eager), "stream launches differ from the eager call"
            t_stream = e0.elapsed_time(e1) * 1e-3 / n
            device_bound = host < 0.8 * t_stream
            t = min(t_graph, t_stream) if device_bound else t_graph
            byts = h.nbytes + 2 * B * K + 4 * B * M
            r[f"B{B}"] = {"us": t * 1e6, "us_graph": t_graph * 1e6, "us_stream": t_stream * 1e6,
                          "host_us": host * 1e6, "gbs": byts / t / 1e9, "frac": byts / t / 1e9 / HBM_PEAK_GBS,
                          "tflops": 2.0 * B * M * K / t / 1e12}
        res[name] = r
    return res


# ------------------------------------------------------------------------------------------------ paged KV (C4)
def _warm(fn, warmup: int, warm_s: float) -> None:
    """Back-to-back launches for at least warm_s seconds (and `warmup` launches) so that the clocks reach the state
    they hold under continuous load."""
    import torch
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < warm_s:
        for _ in range(20):
            fn()
        n += 20
        torch.cuda.synchronize()


def _sustained_time(fn, steps: int, warmup: int, warm_s: float):
    """_warm, then `steps` timed launches, each bracketed by events on the launch stream.
    Returns (wall ms of the timed launches, per-launch ms)."""
    _warm(fn, warmup, warm_s)
    return _events_time(fn, steps, 0, 0.0)


def bench_stream_read(buf, steps: int = 20, warmup: int = 3) -> dict:
    """The device's achievable HBM read bandwidth: cf_stream_read_async (one workgroup per 64 KiB chunk, 16-byte
    non-temporal loads, each byte read once) over `buf` (a uint8 device tensor of >= 2 GB, e.g. the KV pool itself)."""
    import torch
    from chromofold_amd import _abi as A
    A.declare("cf_stream_read_async", A.I32, [A.P, A.U64, A.P, A.P])
    n = (buf.numel() // 16) * 16
    sink = torch.zeros(1, dtype=torch.int32, device=buf.device)
    s = torch.cuda.current_stream().cuda_stream

    def read():
        A.check(A.lib().cf_stream_read_async(buf.data_ptr(), n, sink.data_ptr(), s), "cf_stream_read_async")
    _, per = _events_time(read, steps, warmup)
    t = float(np.median(per)) * 1e-3
    return {"bytes": n, "ms": t * 1e3, "read_gbs": n / t / 1e9}


def bench_cache_peaks(steps: int = 10, warmup: int = 2) -> dict:
    """Read bandwidth of the on-chip levels, as references for the index kernels whose data is L2/LDS resident:
    cf_cache_read_async over 16 MiB (2 MiB per XCD: each XCD's L2 after the first pass; 128 passes) and over 128 MiB
    (beyond the L2s: the Infinity Cache; 16 passes), 2 GiB read per launch; cf_lds_read_async (64 KiB of LDS per
    workgroup, 2 per CU, 64 passes)."""
    import torch
    from chromofold_amd import _abi as A
    A.declare("cf_cache_read_async", A.I32, [A.P, A.U64, A.U32, A.P, A.P])
    A.declare("cf_lds_read_async", A.I32, [A.U32, A.P, A.P])
    A.declare("cf_lds_read_bytes", A.U64, [A.U32])
    L = A.lib()
    s = torch.cuda.current_stream().cuda_stream
    sink = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    res = {}
    for name, nbytes, passes in (("l2_read_gbs", 16 << 20, 128), ("mall_read_gbs", 128 << 20, 16)):
        buf = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda:0")
        fn = lambda: A.check(L.cf_cache_read_async(buf.data_ptr(), nbytes, passes, sink.data_ptr(), s),  # noqa
                             "cf_cache_read_async")
        _, per = _events_time(fn, steps, warmup)
        res[name] = passes * nbytes / (float(np.median(per)) * 1e-3) / 1e9
        del buf
    passes = 64
    _, per = _events_time(lambda: A.check(L.cf_lds_read_async(passes, sink.data_ptr(), s), "cf_lds_read_async"),
                          steps, warmup)
    res["lds_read_gbs"] = int(L.cf_lds_read_bytes(passes)) / (float(np.median(per)) * 1e-3) / 1e9
    return res


def bench_kv(steps: int, warmup: int, context: int = 32768, batch: int = 32, cpu: bool = True,
             check_seqs: int = 8, warm_s: float = 3.0, stream_peak: bool = True, codec: int | None = None) -> dict:
    """Llama-3-8B layer shape (32 q / 8 KV heads, hd 128, 16-token pages), K/V ~ N(0,1) fp32
    generated on the device (seeded), sealed on the device into RANS_HYBRID page groups (per-page-per-head int8
    absmax, rANS) with cf_kv_encode_groups_async; one decode token per sequence per step.
    Gate: the first check_seqs sequences' outputs against the float64 oracle over the pool's own blobs (decoded by
    the oracle), every (sequence, head) row within 1e-3 normwise. The same oracle run on all host threads is the
    CPU baseline (plus its 1-thread figure on one sequence). codec=kv.CODEC_INT8 seals the same data as raw int8
    groups instead (the decode-free codec, 8.03 b/value), to show what the rANS decode costs against raw bytes."""
    import torch
    from chromofold_amd import kv, synth
    codec = kv.CODEC_RANS_HYBRID if codec is None else codec

    H, QH, D = 8, 32, 128
    gqa = QH // H
    t0 = time.perf_counter()
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(synth.SEED_C4 + context)
    K = torch.randn((batch, H, context, D), generator=gen, device="cuda:0")
    V = torch.randn((batch, H, context, D), generator=gen, device="cuda:0")
    Kh = K[0, 0, :1024].cpu().numpy().reshape(-1, 16, D)
    Vh = V[0, 0, :1024].cpu().numpy().reshape(-1, 16, D)
    tables = np.concatenate([t for _ in range(H) for t in (kv.build_table(Kh), kv.build_table(Vh))])
    if codec == kv.CODEC_INT8:
        tables = np.zeros(0, np.uint8)
    kvb = kv.seal_device(codec, K, V, torch.from_numpy(tables).to("cuda:0") if tables.size else None)
    # order-0 entropy of the int8 symbols (sequence 0, every head, K and V; per-page absmax, half to even)
    pg = torch.cat([K[0], V[0]]).reshape(-1, 16 * D)
    sym = torch.round(pg / torch.where(pg.abs().amax(1, keepdim=True) == 0, 1.0, pg.abs().amax(1, keepdim=True) / 127))
    cnt = torch.bincount((sym.clamp(-128, 127) + 128).to(torch.int64).ravel(), minlength=256).double()
    pr = cnt[cnt > 0] / cnt.sum()
    h0 = float(-(pr * torch.log2(pr)).sum())
    del K, V, pg, sym
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t0
    q = torch.randn((batch, QH, D), generator=gen, device="cuda:0")
    qp = torch.full((batch,), context - 1, dtype=torch.int32, device="cuda:0")
    sc = 1.0 / np.sqrt(D)
    out = torch.empty_like(q)
    desc = kvb.desc(q, out, qp, sc)
    kvb.attention(q, out, qp, sc, desc=desc)
    torch.cuda.synchronize()
    res = {"workload": f"{batch} seqs x {context} tokens, 32 q / 8 KV heads, hd {D}", "build_s": t_build,
           "pool_bytes": kvb.pool_bytes}
    if check_seqs > 0:
        import oracle as O
        pool_h = kvb.pool.cpu().numpy()
        offs_h = kvb.group_offsets.cpu().numpy().view(np.uint32)
        toks_h = np.full(batch, context, np.uint32)
        qp_h = np.full(batch, context - 1, np.uint32)
        q_h = q.cpu().numpy()
        got = out.cpu().numpy()
        th = O.num_threads()
        tc0 = time.perf_counter()
        ref = O.kv_pool_attention(pool_h, offs_h, toks_h, qp_h, tables, q_h, H, D, sc, nseq=check_seqs)
        t_all = time.perf_counter() - tc0
        err = np.abs(got[:check_seqs] - ref).max(axis=2) / np.abs(ref).max(axis=2)  # per (sequence, head) row
        res["max_normwise_err"] = float(err.max())
        assert err.max() <= 1e-3, float(err.max())
        if cpu:
            tc1 = time.perf_counter()
            O.kv_pool_attention(pool_h, offs_h, toks_h, qp_h, tables, q_h, H, D, sc, nseq=1, threads=1)
            t_one = time.perf_counter() - tc1
            res["cpu_baseline"] = {
                "value": check_seqs / t_all, "unit": "tokens/s", "cores": th, "kind": "port",
                "sample": f"{check_seqs} sequences x 1 decode token at {context} context (all 8 KV heads): oracle "
                          f"group decode + float64 attention, OpenMP on {th} threads (nproc {os.cpu_count()})",
                "one_thread": {"value": 1.0 / t_one, "unit": "tokens/s", "cores": 1,
                               "sample": f"1 sequence x 1 decode token at {context} context, 1 thread"}}
        del pool_h
    wall, per = _sustained_time(lambda: kvb.attention(q, out, qp, sc, desc=desc), steps, warmup, warm_s)
    t_step = float(np.mean(per)) * 1e-3
    # algorithmic bytes per step: every visible page blob (payload + header + states), tables once, page table,
    # queries and outputs
    step_bytes = kvb.pool_bytes + tables.size + batch * H * (context // 64) * 4 + 2 * q.numel() * 4
    values = 2 * batch * H * context * D
    res.update({
        "tokens_per_s": batch / t_step, "ms_per_step": wall / steps, "kernel_ms": t_step * 1e3,
        "kernel_ms_min": float(np.min(per)), "kernel_ms_max": float(np.max(per)),
        "bits_per_value": kvb.pool_bytes * 8.0 / values, "int8_bits_per_value": 8.0 + 8.0 * 64 / (16 * D * 4 * 2),
        "symbol_entropy_bits": h0,
        "ratio_vs_bf16": (values * 2.0) / kvb.pool_bytes,
        "roofline": {"bound": "hbm", "achieved": step_bytes / t_step / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": step_bytes / t_step / 1e9 / HBM_PEAK_GBS,
                     "traffic": MEASURED_TRAFFIC.get(("kv", context, batch))},
        "step_bytes": step_bytes,
    })
    if stream_peak:
        sr = bench_stream_read(kvb.pool)
        res["hbm_read_peak_gbs"] = sr["read_gbs"]
        res["frac_of_read_peak"] = res["roofline"]["achieved"] / sr["read_gbs"]
    return res


# ------------------------------------------------------------------------------------------------ device sealing
def bench_seal(steps: int, warmup: int, cpu: bool = True, seqs: int = 32, tokens: int = 4096) -> dict:
    """Sealing on the device (cf_kv_encode_groups_async): the C4 shape's prompt KV (32 sequences x 4096 tokens x 8
    KV heads, hd 128, fp32, already in HBM) quantised and rANS-coded into one pool per call. Gate: the first 64
    groups' bytes and offsets equal the host encoder's on the same pages. CPU baseline: the host encoder
    (cf_kv_encode_groups, all host threads) on a 2048-group sample."""
    import torch
    from chromofold_amd import _abi as A
    from chromofold_amd import kv, synth

    H, D = 8, 128
    pages = seqs * H * tokens // 16
    ngroups = pages // 4
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(synth.SEED_C4 + 7)
    K = torch.randn((pages, 16, D), generator=gen, device="cuda:0", dtype=torch.float32)
    V = torch.randn((pages, 16, D), generator=gen, device="cuda:0", dtype=torch.float32)
    Ks = K[:256].cpu().numpy()
    Vs = V[:256].cpu().numpy()
    tables = np.concatenate([t for h in range(H) for t in (kv.build_table(Ks[32 * h:32 * h + 32]),
                                                           kv.build_table(Vs[32 * h:32 * h + 32]))])
    first = np.arange(ngroups, dtype=np.int64) * 4
    heads = ((np.arange(ngroups) // (tokens // 64)) % H).astype(np.int32)
    d_first = torch.from_numpy(first).to("cuda:0")
    d_counts = torch.full((ngroups,), 4, dtype=torch.int32, device="cuda:0")
    d_heads = torch.from_numpy(heads).to("cuda:0")
    d_tab = torch.from_numpy(tables).to("cuda:0")
    cap = ngroups * int(A.lib().cf_kv_group_blob_max_bytes(kv.CODEC_RANS_HYBRID, D))
    pool = torch.empty(cap, dtype=torch.uint8, device="cuda:0")
    ws = torch.empty(int(A.lib().cf_kv_encode_groups_workspace_bytes(kv.CODEC_RANS_HYBRID, D, ngroups, 2 * H)),
                     dtype=torch.uint8, device="cuda:0")

    cont = ((np.arange(ngroups) % (tokens // 64)) % 2).astype(np.uint8)  # groups 2k, 2k + 1 of a head: one chain
    d_cont = torch.from_numpy(cont).to("cuda:0")

    def seal():
        return kv.encode_groups_device(kv.CODEC_RANS_HYBRID, K, V, D, d_tab, d_first, d_counts, pool, 0, d_heads,
                                       None, ws, continues=d_cont)

    r = seal()
    torch.cuda.synchronize()
    assert int(r.status.item()) == 0
    end = int(r.pool_end.item())
    n_chk = 64
    host, hoff = kv.encode_groups(kv.CODEC_RANS_HYBRID, Ks, Vs, D, tables, first[:n_chk], np.full(n_chk, 4),
                                  heads[:n_chk].astype(np.uint32), continues=cont[:n_chk])
    assert np.array_equal(r.offsets[:n_chk].cpu().numpy().view(np.uint32), hoff), "device offsets != host"
    assert np.array_equal(pool[:host.size].cpu().numpy(), host), "device-sealed bytes != host encoder bytes"
    wall, per = _events_time(seal, steps, warmup)
    t = float(np.mean(per)) * 1e-3
    in_bytes = 2 * K.numel() * 4
    res = {"workload": f"{seqs} seqs x {tokens} tokens x {H} KV heads, hd {D}: {ngroups} groups per call",
           "ms_per_call": t * 1e3, "groups_per_s": ngroups / t, "tokens_per_s": seqs * tokens / t,
           "fp32_in_gbs": in_bytes / t / 1e9, "pool_bytes": end,
           "hbm_frac": (in_bytes + end) / t / 1e9 / HBM_PEAK_GBS}
    if cpu:
        n = 2048
        Kh, Vh = K[:4 * n].cpu().numpy(), V[:4 * n].cpu().numpy()
        th = min(16, os.cpu_count() or 1)  # the box's CPU share for one GPU
        t0 = time.perf_counter()
        kv.encode_groups(kv.CODEC_RANS_HYBRID, Kh, Vh, D, tables, first[:n], np.full(n, 4),
                         heads[:n].astype(np.uint32), threads=th, continues=cont[:n])
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": n / dt, "unit": "groups/s", "cores": th, "kind": "port",
                               "sample": f"{n} groups with the library's host encoder on {th} threads"}
    return res


# ------------------------------------------------------------------------------------- gathers (sparse consumers)
def bench_gather(steps: int, warmup: int, dim: int = 128, nq: int = 1 << 20) -> dict:
    """Embedding-row gathers through the C1 index (1M Zipf tokens, vocab 32000, GPU-built RRR wavelet): for 1M
    random positions, out[q] = emb[token[pos[q]]] with emb [32000, 128] fp32. Fused (cf_sparse_gather_fused_async:
    access + row copy in one kernel) against decode-all + gather (cf_sparse_decode_all_async once, then
    cf_sparse_gather_async per step). Gate: the closed form emb[tok[pos]]. Algorithmic HBM bytes per call: the
    positions and the output rows (the 16 MB table and the index stay in L2/MALL)."""
    import ctypes as C
    import torch
    from chromofold_amd import _abi as A
    from chromofold_amd import synth
    from chromofold_amd.search import build_rrrw, u32_dev

    n, vocab = 1 << 20, 32000
    tok = synth.zipf_tokens(n, vocab, 1.1, synth.SEED_C1)
    idx, _ = build_rrrw(torch.from_numpy(tok.view(np.int32)).to("cuda:0"), 15)
    rng = np.random.default_rng(synth.SEED_C1 + 9)
    pos = rng.integers(0, n, nq).astype(np.uint32)
    emb = torch.randn((vocab, dim), device="cuda:0", generator=torch.Generator(device="cuda:0").manual_seed(3))
    dpos = u32_dev(pos)
    out = torch.empty((nq, dim), device="cuda:0")
    ids = torch.empty(n, dtype=torch.int32, device="cuda:0")
    L = A.lib()
    v = idx.view()
    for name, args in (("cf_sparse_gather_fused_async", [A.cf_rrrw_view, A.P, C.c_int, A.P, A.P, C.c_size_t, A.P]),
                       ("cf_sparse_decode_all_async", [A.cf_rrrw_view, A.P, C.c_size_t, A.P]),
                       ("cf_sparse_gather_async", [A.P, A.P, C.c_int, A.P, A.P, C.c_size_t, A.P])):
        A.declare(name, A.I32, args)
    s = torch.cuda.current_stream().cuda_stream

    def fused():
        A.check(L.cf_sparse_gather_fused_async(v, emb.data_ptr(), dim, dpos.data_ptr(), out.data_ptr(), nq, s),
                "cf_sparse_gather_fused_async")

    def fused_lines():
        idx.gather_fused_lines_into(emb, dpos, out, stream=torch.cuda.current_stream())

    def fused_quads():
        idx.gather_fused_quads_into(emb, dpos, out, stream=torch.cuda.current_stream())

    def via_ids():
        A.check(L.cf_sparse_gather_async(ids.data_ptr(), emb.data_ptr(), dim, dpos.data_ptr(), out.data_ptr(), nq, s),
                "cf_sparse_gather_async")

    fused()
    torch.cuda.synchronize()
    chk = rng.integers(0, nq, 4096)
    ref = emb[torch.from_numpy(tok[pos[chk]].astype(np.int64)).to("cuda:0")]
    assert torch.equal(out[torch.from_numpy(chk).to("cuda:0")], ref), "fused gather != emb[tok[pos]]"
    _, per_f = _events_time(fused, steps, warmup)
    out.fill_(float("nan"))
    fused_lines()
    torch.cuda.synchronize()
    assert torch.equal(out[torch.from_numpy(chk).to("cuda:0")], ref), "fused gather (lines) != emb[tok[pos]]"
    _, per_fl = _events_time(fused_lines, steps, warmup)
    idx.build_quads(n)
    out.fill_(float("nan"))
    fused_quads()
    torch.cuda.synchronize()
    assert torch.equal(out[torch.from_numpy(chk).to("cuda:0")], ref), "fused gather (quads) != emb[tok[pos]]"
    _, per_fq = _events_time(fused_quads, steps, warmup)
    A.check(L.cf_sparse_decode_all_async(v, ids.data_ptr(), n, s), "cf_sparse_decode_all_async")
    _, per_d = _events_time(lambda: A.check(L.cf_sparse_decode_all_async(v, ids.data_ptr(), n, s), "decode_all"),
                            steps, warmup)
    _, per_g = _events_time(via_ids, steps, warmup)
    torch.cuda.synchronize()
    assert torch.equal(out[torch.from_numpy(chk).to("cuda:0")], ref), "gather via ids != emb[tok[pos]]"
    tf, tfl, tfq, td, tg = (float(np.mean(p)) * 1e-3 for p in (per_f, per_fl, per_fq, per_d, per_g))
    step_bytes = nq * 4 + nq * dim * 4
    return {"workload": f"{nq} positions into the C1 index, rows of {dim} fp32 from a {vocab}-row table",
            "fused_ms": tf * 1e3, "fused_mqs": nq / tf / 1e6, "fused_gbs": step_bytes / tf / 1e9,
            "fused_roofline_frac": step_bytes / tf / 1e9 / HBM_PEAK_GBS,
            "fused_lines_ms": tfl * 1e3, "fused_lines_gbs": step_bytes / tfl / 1e9,
            "fused_lines_roofline_frac": step_bytes / tfl / 1e9 / HBM_PEAK_GBS,
            "fused_quads_ms": tfq * 1e3, "fused_quads_gbs": step_bytes / tfq / 1e9,
            "fused_quads_roofline_frac": step_bytes / tfq / 1e9 / HBM_PEAK_GBS,
            "decode_all_ms": td * 1e3, "gather_via_ids_ms": tg * 1e3,
            "decode_all_plus_gather_ms": (td + tg) * 1e3}


# ------------------------------------------------------------------------------------------------ int4 nibble pages
def _d2h(ptr: int, nbytes: int) -> np.ndarray:
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    out = np.empty(nbytes, np.uint8)
    assert hip.hipMemcpy(out.ctypes.data, ptr, nbytes, 2) == 0  # device to host
    return out


def _nib_dequant(payload: np.ndarray, scales: np.ndarray, bs: int) -> np.ndarray:
    sym = np.empty(payload.size * 2, np.int64)
    sym[0::2] = payload & 0x0F
    sym[1::2] = payload >> 4
    return (sym - 8) * scales.astype(np.float64)[np.arange(sym.size) // bs]


def bench_nibble(steps: int, warmup: int, cpu: bool = True, seqs: int = 32, tokens: int = 32768, page: int = 64,
                 bs: int = 32) -> dict:
    """Batched decode over int4 nibble pages through the multi-sequence resolver (cf_ms_cuda_execute_batch_async):
    C4 shape (32 sequences x 32768 tokens, 8 KV / 32 q heads, hd 128), pages of 64 tokens sealed on the device by
    the seal engine (block 32), published to 32 resolver sequences; one step = one batch of 32 decode items (one
    attention launch + one merge launch). Gate: sequence 0 against a float64 numpy softmax over its pages'
    dequantised bytes (read back from HBM). CPU baseline: the oracle's attention on a 4096-token sample."""
    import ctypes as C
    import torch
    from chromofold_amd import _abi as A
    from chromofold_amd import sealkv as SK

    H, QH, D = 8, 32, 128
    gqa = QH // H
    sc = 1.0 / np.sqrt(D)
    npg = tokens // page
    eng = SK.SealEngine(seqs, H, QH, D, page, bs)
    res_ = SK.MsResolver(1, H, QH, D, page)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(0x5EA1)
    t0 = time.perf_counter()
    for s in range(seqs):
        res_.create(s)
        for p in range(npg):
            kv_ = torch.randn((2, page, H, D), generator=gen, device="cuda:0")
            eng.stage(s, p * page, kv_[0], kv_[1])
            eng.seal(s)
        for d in eng.pages(s):
            res_.publish(s, 0, d)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    q = torch.randn((seqs, 1, QH, D), generator=gen, device="cuda:0")
    out = torch.empty_like(q)
    arr = (SK.cf_ms_batch_item * seqs)()
    for s in range(seqs):
        op, ot, ots, ohs, oes = SK._out_args(out[s])
        arr[s] = SK.cf_ms_batch_item(s, 0, SK.tensor_view(q[s]), op, ot, ots, ohs, oes, tokens - 1, sc, 0)
    L = A.lib()
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        if L.cf_ms_cuda_execute_batch_async(res_.h, arr, seqs, stream) != 0:
            raise RuntimeError(L.cf_ms_cuda_last_error(res_.h).decode())

    step()
    torch.cuda.synchronize()
    # gate: sequence 0 in float64 from the sealed bytes
    descs = eng.pages(0)
    vals = page * H * D
    Kd = np.concatenate([_nib_dequant(_d2h(d.key_payload, vals // 2), _d2h(d.key_scales, vals // bs * 4).view(
        np.float32), bs) for d in descs]).reshape(tokens, H, D)
    Vd = np.concatenate([_nib_dequant(_d2h(d.value_payload, vals // 2), _d2h(d.value_scales, vals // bs * 4).view(
        np.float32), bs) for d in descs]).reshape(tokens, H, D)
    qh = q[0, 0].double().cpu().numpy()
    ref = np.empty((QH, D))
    for h in range(QH):
        sco = Kd[:, h // gqa] @ qh[h] * sc
        w = np.exp(sco - sco.max())
        ref[h] = w @ Vd[:, h // gqa] / w.sum()
    got = out[0, 0].double().cpu().numpy()
    err = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    assert err <= 1e-3, err
    wall, per = _events_time(step, steps, warmup)
    torch.cuda.synchronize()
    res_.reclaim()
    t = float(np.mean(per)) * 1e-3
    page_bytes = sum(d.resident_bytes for s in range(seqs) for d in eng.pages(s))
    step_bytes = page_bytes + seqs * npg * C.sizeof(SK.cf_device_page_descriptor) + q.numel() * 4 * 2
    r = {"workload": f"{seqs} seqs x {tokens} tokens, int4 nibble pages of {page} tokens (block {bs}), 32 q / 8 kv "
                     f"heads, hd {D}, one batch of {seqs} decode items per step",
         "tokens_per_s": seqs / t, "ms_per_step": t * 1e3, "page_bytes": page_bytes,
         "bits_per_value": page_bytes * 8 / (2 * seqs * tokens * H * D), "hbm_gbs": step_bytes / t / 1e9,
         "roofline_frac": step_bytes / t / 1e9 / HBM_PEAK_GBS, "seq0_normwise_err": err, "build_s": build_s}
    if cpu:
        import oracle as O
        ns = 4096
        pages = []
        for i, d in enumerate(descs[: ns // page]):
            pages.append(O.NibPage(_d2h(d.key_payload, vals // 2), _d2h(d.value_payload, vals // 2),
                                   _d2h(d.key_scales, vals // bs * 4).view(np.float32),
                                   _d2h(d.value_scales, vals // bs * 4).view(np.float32), i * page, page))
        qn = q[0].cpu().numpy()
        t1 = time.perf_counter()
        O.nib_attention(pages, bs, qn, ns - 1, H, gqa, sc)
        dt = (time.perf_counter() - t1) * tokens / ns
        r["cpu_baseline"] = {"value": 1.0 / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
                             "sample": f"oracle attention (float64) of one decode token over {ns} tokens, scaled "
                                       f"to {tokens}"}
    res_.close()
    eng.close()
    return r


# ------------------------------------------------------------------------------------------------ long context (C5)
def bench_seam(steps: int, warmup: int, shapes=((64, 4096), (64, 65536), (128, 4096), (128, 65536))) -> dict:
    """The reference seam (cf_kv_paged_attention_async) through the llama adapter (cf_llama_kv_*), at the shape of
    the reference's own seam benchmark (reference product/native-kv-performance.json: Qwen2.5-0.5B-derived
    attention, 2 KV / 14 query heads, 64 query tokens per call, contexts 4096-65536, head_dim 64 and 128): int4
    fixed-width pages of 32 tokens, 65536 tokens = 4096 pages = the seam's per-launch page limit. One call = the 64
    query tokens at the end of the context, causal. Gate: the last query row against the float64 oracle over the
    fixture-quantised pages. The reference published 2528 us for its final kernel on an RTX 2080 Ti
    (native-kv-performance.json:10)."""
    import torch
    import oracle as O
    from chromofold_amd import llama

    out = {"workload": "llama adapter seam: 2 KV / 14 q heads, 64 queries, int4 pages of 32 tokens",
           "reference_us": 2528, "reference_hw": "RTX 2080 Ti (native-kv-performance.json:10)"}
    kvh, qh, gqa, qn, ps = 2, 14, 7, 64, 32
    for hd, n in shapes:
        ad = llama.KvAdapter(llama.options(1, kvh, qh, hd, ps, gqa, 4))
        rng = np.random.default_rng(0x5EA + n + hd)
        keys, vals = [], []
        for h in range(kvh):
            k = rng.standard_normal((n, hd)).astype(np.float32)
            v = rng.standard_normal((n, hd)).astype(np.float32)
            ad.append(0, h, 0, k, v)
            keys.append(k)
            vals.append(v)
        q = torch.from_numpy(rng.standard_normal((qn, qh, hd)).astype(np.float32)).to("cuda:0")
        o = torch.empty_like(q)
        s = torch.cuda.current_stream().cuda_stream
        sc = 1.0 / np.sqrt(hd)
        run = lambda: ad.attention(0, q.data_ptr(), o.data_ptr(), qn, qh, gqa, n - qn, sc, 0, s)  # noqa: E731
        run()
        torch.cuda.synchronize()
        pages = []
        for h in range(kvh):
            for p0 in range(0, n, ps):
                *_, kd, vd = O.kv_fixture_quantize(keys[h][p0:p0 + ps], vals[h][p0:p0 + ps], 4)
                pages.append((h, p0, kd, vd))
        ref, _ = O.paged_attention_f64(q[qn - 1].cpu().numpy(), qh, kvh, hd, gqa, n - 1, 0, sc, pages)
        got = o[qn - 1].cpu().numpy()
        err = float(np.abs(got - ref).max())
        assert err <= 2e-4, err
        _, per = _events_time(run, steps, warmup)
        t = float(np.median(per)) * 1e-3
        st = ad.stats()
        nbytes = st.compressed_bytes + st.descriptor_bytes + 2 * q.numel() * 4
        out[f"hd{hd}_n{n}"] = {"us": t * 1e6, "compressed_bytes": int(st.compressed_bytes),
                               "gbs": nbytes / t / 1e9, "roofline_frac": nbytes / t / 1e9 / HBM_PEAK_GBS,
                               "x_vs_reference": 2528e-6 / t, "max_abs_err_last_row": err}
        ad.close()
        del pages
    out["rans_pages"] = bench_seam_rans(steps, warmup)
    return out


def bench_seam_c4(steps: int, warmup: int, context: int = 32768, batch: int = 32) -> dict:
    """The headline configuration through the unchanged reference seam (the llama.cpp integration's call,
    reference integrations/llama.cpp/chromofold_kv_adapter.cpp:127): C4's 32 sequences x 32768 tokens, 8 KV / 32 q
    heads, hd 128, every 64 tokens of a (sequence, KV head) one self-coded RANS_HYBRID group (a chain start, the
    seam's rANS page tag), sealed on the device. 8 x 512 = 4096 pages per sequence = the seam's per-launch page
    limit (reference include/chromofold/kv_cuda.h:13), so one step is 32 cf_kv_paged_attention_async calls, one
    per sequence, each with its decode token's 32 query heads. Gate: sequence 0's output against the float64 oracle
    decoding the pool's own blobs."""
    import ctypes as C
    import torch
    import oracle as O
    from chromofold_amd import _abi as A
    from chromofold_amd import kv, legacy, synth

    H, QH, D = 8, 32, 128
    gqa = QH // H
    ngr = context // 64
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(synth.SEED_C4 + context)
    K = torch.randn((batch, H, context, D), generator=gen, device="cuda:0")
    V = torch.randn((batch, H, context, D), generator=gen, device="cuda:0")
    Kh = K[0, 0, :1024].cpu().numpy().reshape(-1, 16, D)
    Vh = V[0, 0, :1024].cpu().numpy().reshape(-1, 16, D)
    tables = np.concatenate([t for _ in range(H) for t in (kv.build_table(Kh), kv.build_table(Vh))])
    d_tab = torch.from_numpy(tables).to("cuda:0")
    n = batch * H * ngr
    g = torch.arange(n, device="cuda:0", dtype=torch.int64)
    first = (g // ngr) * (context // 16) + (g % ngr) * 4
    heads = ((g // ngr) % H).to(torch.int32)
    cap = int(A.lib().cf_kv_group_blob_max_bytes(kv.CODEC_RANS_HYBRID, D)) * n
    pool = torch.empty(cap, dtype=torch.uint8, device="cuda:0")
    r = kv.encode_groups_device(kv.CODEC_RANS_HYBRID, K.view(-1, 16, D), V.view(-1, 16, D), D, d_tab, first,
                                torch.full((n,), 4, dtype=torch.int32, device="cuda:0"), pool, 0, heads,
                                continues=torch.zeros(n, dtype=torch.uint8, device="cuda:0"))
    st, end = int(r.status.item()), int(r.pool_end.item())
    assert st == 0, st
    del K, V
    offs = r.offsets.cpu().numpy().view(np.uint32).astype(np.uint64).reshape(batch, H, ngr)
    page_dt = np.dtype({"names": ["k_words", "k_lut", "v_lut", "token_begin", "token_count", "head_dim",
                                  "block_size", "zero_point", "kv_head"],
                        "formats": ["<u8", "<u8", "<u8", "<u4", "<u4", "<u4", "<u4", "<u4", "<u4"],
                        "offsets": [0, 16, 48, 64, 68, 72, 76, 88, 92], "itemsize": C.sizeof(A.cf_kv_device_page)})
    descs = np.zeros((batch, H * ngr), page_dt)
    hh = np.repeat(np.arange(H, dtype=np.uint64), ngr)
    gg = np.tile(np.arange(ngr, dtype=np.uint32), H)
    base, tb = pool.data_ptr(), d_tab.data_ptr()
    for s_ in range(batch):
        d_ = descs[s_]
        d_["k_words"] = base + offs[s_].reshape(-1) * 16
        d_["k_lut"] = tb + hh * (2 * kv.TABLE_BYTES)
        d_["v_lut"] = tb + hh * (2 * kv.TABLE_BYTES) + kv.TABLE_BYTES
        d_["token_begin"], d_["token_count"], d_["head_dim"], d_["block_size"] = 64 * gg, 64, D, 64
        d_["zero_point"], d_["kv_head"] = 128, hh.astype(np.uint32)
    d_descs = torch.from_numpy(descs.view(np.uint8)).to("cuda:0")
    q = torch.randn((batch, 1, QH, D), generator=gen, device="cuda:0")
    out = torch.empty_like(q)
    sc = 1.0 / np.sqrt(D)
    row = descs.itemsize * H * ngr
    ds = []
    for s_ in range(batch):
        d = A.cf_kv_paged_attention_desc()
        d.struct_size, d.abi_version = C.sizeof(A.cf_kv_paged_attention_desc), legacy.CF_KV_CUDA_ABI_VERSION
        d.pages, d.page_count = d_descs.data_ptr() + s_ * row, H * ngr
        d.kv_head_count, d.query_head_count, d.gqa_group_size = H, QH, gqa
        d.queries, d.output = q[s_].data_ptr(), out[s_].data_ptr()
        d.query_token_begin, d.query_count, d.head_dim, d.softmax_scale = context - 1, 1, D, sc
        ds.append(d)
    L = A.lib()
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        for d in ds:
            A.check(L.cf_kv_paged_attention_async(C.byref(d), stream), "cf_kv_paged_attention_async")

    step()
    torch.cuda.synchronize()
    got = out[0, 0].cpu().numpy()
    ref = O.kv_pool_attention(pool[:end].cpu().numpy(), offs[:1].astype(np.uint32), np.full(1, context, np.uint32),
                              np.full(1, context - 1, np.uint32), tables, q[:1, 0].cpu().numpy(), H, D, sc, nseq=1)
    err = float((np.abs(got - ref[0]).max(axis=1) / np.abs(ref[0]).max(axis=1)).max())
    assert err <= 1e-3, err
    _, per = _events_time(step, steps, warmup)
    t = float(np.mean(per)) * 1e-3
    step_bytes = end + tables.size + d_descs.numel() + 2 * q.numel() * 4
    return {"workload": f"reference seam at C4: {batch} seqs x {context} tokens, 32 q / 8 KV heads, hd {D}, "
                        f"{H * ngr} self-coded 64-token rANS pages per call, {batch} calls per step",
            "tokens_per_s": batch / t, "ms_per_step": t * 1e3, "us_per_call": t * 1e6 / batch,
            "pool_bytes": end, "bits_per_value": end * 8.0 / (2 * batch * H * context * D),
            "gbs": step_bytes / t / 1e9, "roofline_frac": step_bytes / t / 1e9 / HBM_PEAK_GBS,
            "max_normwise_err_seq0": err}


def bench_seam_rans(steps: int, warmup: int, hd: int = 128, n: int = 65536) -> dict:
    """The same seam call over rANS pages (the seam's rANS tag, kv_cuda.h: fixed_code_length == 0 and
    k_max_code_length == 0): every 64 tokens of a KV head one kv_codec_ext.h RANS_HYBRID group coded on its own,
    the head's pages sharing one K and one V table. Gate: the last query row against the float64 oracle over the
    values the oracle decodes from every group."""
    import ctypes as C
    import torch
    import oracle as O
    from chromofold_amd import _abi as A
    from chromofold_amd import kv, legacy

    kvh, qh, gqa, qn = 2, 14, 7, 64
    rng = np.random.default_rng(0x5EB + n + hd)
    ng = n // 64
    descs = (A.cf_kv_device_page * (kvh * ng))()
    keep, pages, coded = [], [], 0
    for h in range(kvh):
        K = rng.standard_normal((n // 16, 16, hd)).astype(np.float32)
        V = rng.standard_normal((n // 16, 16, hd)).astype(np.float32)
        tables = np.concatenate([kv.build_table(K[:256]), kv.build_table(V[:256])])
        blob, offs = kv.encode_groups(kv.CODEC_RANS_HYBRID, K, V, hd, tables, np.arange(ng, dtype=np.uint64) * 4,
                                      np.full(ng, 4, np.uint32))
        coded += blob.size + tables.size
        dpool = torch.from_numpy(blob).to("cuda:0")
        dtab = torch.from_numpy(tables).to("cuda:0")
        keep += [dpool, dtab]
        ends = list(offs[1:].astype(np.int64) * 16) + [blob.size]
        for g in range(ng):
            d = descs[h * ng + g]
            d.k_words = dpool.data_ptr() + int(offs[g]) * 16
            d.k_lut, d.v_lut = dtab.data_ptr(), dtab.data_ptr() + kv.TABLE_BYTES
            d.token_begin, d.token_count, d.head_dim, d.block_size = 64 * g, 64, hd, 64
            d.zero_point, d.kv_head = 128, h
            ks, vs, ksc, vsc, _ = O.kv_decode_group(blob[int(offs[g]) * 16:ends[g]], tables, 0, hd)
            kd = np.concatenate([(ks[p].astype(np.float32) - 128) * ksc[p] for p in range(4)])
            vd = np.concatenate([(vs[p].astype(np.float32) - 128) * vsc[p] for p in range(4)])
            pages.append((h, 64 * g, kd, vd))
    dd = torch.from_numpy(np.frombuffer(bytes(descs), np.uint8).copy()).to("cuda:0")
    q = torch.from_numpy(rng.standard_normal((qn, qh, hd)).astype(np.float32)).to("cuda:0")
    o = torch.empty_like(q)
    desc = A.cf_kv_paged_attention_desc()
    desc.struct_size, desc.abi_version = C.sizeof(A.cf_kv_paged_attention_desc), legacy.CF_KV_CUDA_ABI_VERSION
    desc.pages, desc.page_count, desc.kv_head_count = dd.data_ptr(), kvh * ng, kvh
    desc.query_head_count, desc.gqa_group_size = qh, gqa
    desc.queries, desc.output = q.data_ptr(), o.data_ptr()
    desc.query_token_begin, desc.query_count, desc.head_dim = n - qn, qn, hd
    desc.softmax_scale = 1.0 / np.sqrt(hd)
    s = torch.cuda.current_stream().cuda_stream
    run = lambda: A.check(A.lib().cf_kv_paged_attention_async(C.byref(desc), s), "cf_kv_paged_attention_async")  # noqa: E731
    run()
    torch.cuda.synchronize()
    ref, _ = O.paged_attention_f64(q[qn - 1].cpu().numpy(), qh, kvh, hd, gqa, n - 1, 0, desc.softmax_scale, pages)
    err = float(np.abs(o[qn - 1].cpu().numpy() - ref).max())
    assert err <= 2e-4, err
    _, per = _events_time(run, steps, warmup)
    t = float(np.median(per)) * 1e-3
    nbytes = coded + C.sizeof(A.cf_kv_device_page) * kvh * ng + 2 * q.numel() * 4
    del keep
    return {"workload": f"seam over rANS pages: 2 KV / 14 q heads, 64 queries, hd {hd}, {n} tokens, one self-coded "
                        "64-token RANS_HYBRID group per page, one K and one V table per head",
            "us": t * 1e6, "coded_bytes": coded, "bits_per_value": 8.0 * coded / (2 * kvh * n * hd),
            "gbs": nbytes / t / 1e9, "roofline_frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "max_abs_err_last_row": err}


def bench_runtime(steps: int, warmup: int, items: int = 32, context: int = 4096, kvh: int = 8, gqa: int = 4,
                  hd: int = 128, page: int = 32, block: int = 32) -> dict:
    """The batched-items decode contract (cf_attention_execute_async, reference production_attention.h): `items`
    decode requests in one call, each over its own device table of `context / page` two's-complement int4 pages
    ([token][kv head][dim], one scale per `block` values of a row), fp32 query and output, no tail. Pages hold
    random nibbles and scales generated on the device. Gate: item 0 against the float64 oracle."""
    import ctypes as C
    import torch
    import oracle as O
    from chromofold_amd import sealkv as S

    qh, npg = kvh * gqa, context // page
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(0xA77E)
    pay_bytes = page * kvh * hd // 2
    nsc = page * kvh * ((hd + block - 1) // block)
    kp = torch.randint(0, 256, (items, npg, pay_bytes), generator=gen, device="cuda:0", dtype=torch.uint8)
    vp = torch.randint(0, 256, (items, npg, pay_bytes), generator=gen, device="cuda:0", dtype=torch.uint8)
    ks = torch.rand((items, npg, nsc), generator=gen, device="cuda:0") * 0.3 + 0.05
    vs = torch.rand((items, npg, nsc), generator=gen, device="cuda:0") * 0.3 + 0.05
    q = torch.randn((items, qh, hd), generator=gen, device="cuda:0")
    out = torch.full_like(q, float("nan"))
    tables = []
    arr = (S.cf_attention_batch_item * items)()
    for i in range(items):
        descs = (S.cf_device_page_descriptor * npg)()
        for p in range(npg):
            d = descs[p]
            d.key_payload, d.value_payload = kp[i, p].data_ptr(), vp[i, p].data_ptr()
            d.key_scales, d.value_scales = ks[i, p].data_ptr(), vs[i, p].data_ptr()
            d.token_begin, d.token_count, d.kv_head_count, d.head_dim, d.block_size = p * page, page, kvh, hd, block
        t = torch.frombuffer(bytearray(descs), dtype=torch.uint8).to("cuda:0")
        tables.append(t)
        it = arr[i]
        it.sequence_id, it.layer = i, 0
        it.query = S.cf_device_tensor_view(q[i].data_ptr(), S.CF_DEVICE_F32, 1, qh, hd, 0, hd * 4, 4, 0)
        it.output, it.output_type = out[i].data_ptr(), S.CF_DEVICE_F32
        it.output_head_stride_bytes, it.output_element_stride_bytes = hd * 4, 4
        it.query_token_begin, it.softmax_scale = context, 1.0 / np.sqrt(hd)
        it.sealed_pages, it.sealed_page_count = t.data_ptr(), npg
    rt = S.AttentionRuntime(1, kvh, qh, hd, gqa=gqa, page_size=page, block_size=block)
    rt.execute(arr)
    torch.cuda.synchronize()
    pages = [O.RtPage(kp[0, p].cpu().numpy(), vp[0, p].cpu().numpy(), ks[0, p].cpu().numpy(), vs[0, p].cpu().numpy(),
                      p * page, page, hd, block) for p in range(npg)]
    ref = O.rt_attention_f64(q[0].cpu().numpy(), kvh, gqa, context, 0, 1.0 / np.sqrt(hd), pages)
    got = out[0].double().cpu().numpy()
    err = float((np.abs(got - ref).max(axis=1) / np.abs(ref).max(axis=1)).max())
    assert err <= 1e-3, err
    _, per = _events_time(lambda: rt.execute(arr), steps, warmup)
    t = float(np.median(per)) * 1e-3
    nbytes = (kp.numel() + vp.numel() + 4 * (ks.numel() + vs.numel()) + items * npg * C.sizeof(S.cf_device_page_descriptor)
              + 2 * q.numel() * 4)
    rt.close()
    del tables
    return {"workload": f"{items} items x {context} tokens, {qh} q / {kvh} KV heads, hd {hd}, int4 pages of {page} "
                        f"tokens, scale blocks of {block}",
            "us": t * 1e6, "tokens_per_s": items / t, "bytes": int(nbytes), "gbs": nbytes / t / 1e9,
            "roofline_frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "max_normwise_err_item0": err}


def bench_c5(steps: int, warmup: int) -> dict:
    """C4 shapes (8 KV / 32 q heads, hd 128, rANS-hybrid pages). (a) 256 sequences sharing one 8192-token prefix
    (stored once, referenced by every sequence's page table) plus 512 unique tokens each; (b) 4 sequences x 131072
    tokens. One decode token per sequence per step. Gate: the fp64 oracle on one sequence of (a) and on KV head 0
    of one sequence of (b)."""
    import torch
    import oracle as O
    from chromofold_amd import kv, synth

    H, QH, D = 8, 32, 128
    gqa = QH // H
    sc = 1.0 / np.sqrt(D)
    res = {}
    rng = np.random.default_rng(synth.SEED_C5)
    K0 = rng.standard_normal((H, 1024, D), dtype=np.float32)
    V0 = rng.standard_normal((H, 1024, D), dtype=np.float32)
    tables = np.concatenate([t for h in range(H) for t in (kv.build_table(K0[h].reshape(-1, 16, D)),
                                                           kv.build_table(V0[h].reshape(-1, 16, D)))])

    def run(kvb, S, T, qp, shared_groups=0):
        q = torch.from_numpy(rng.standard_normal((S, QH, D), dtype=np.float32)).to("cuda:0")
        dqp = torch.from_numpy(qp.view(np.int32)).to("cuda:0")
        out = torch.empty_like(q)
        desc = kvb.desc(q, out, dqp, sc, shared_groups=shared_groups)
        kvb.attention(q, out, dqp, sc, desc=desc, shared_groups=shared_groups)
        torch.cuda.synchronize()
        _, per = _events_time(lambda: kvb.attention(q, out, dqp, sc, desc=desc, shared_groups=shared_groups), steps,
                              warmup)
        return q.cpu().numpy(), out.cpu().numpy(), float(np.mean(per)) * 1e-3

    # (a) shared prefix
    S, P, U = 256, 8192, 512
    T = P + U
    seeds = rng.integers(0, 2 ** 63, size=S)
    prefix = (rng.standard_normal((H, P, D), dtype=np.float32), rng.standard_normal((H, P, D), dtype=np.float32))

    def src_a(s):
        g = np.random.default_rng(int(seeds[s]))
        Ks = np.empty((H, T, D), np.float32)
        Vs = np.empty((H, T, D), np.float32)
        if s == 0:
            Ks[:, :P], Vs[:, :P] = prefix
        else:  # the prefix groups of s > 0 come from sequence 0's blobs and are never encoded from here
            Ks[:, :P] = 0.0
            Vs[:, :P] = 0.0
        Ks[:, P:] = g.standard_normal((H, U, D), dtype=np.float32)
        Vs[:, P:] = g.standard_normal((H, U, D), dtype=np.float32)
        return Ks, Vs

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from kv_helpers import decoded_pages, normwise_err
    logical = 2.0 * S * H * T * D * 2  # bf16 bytes of every sequence's full KV
    # The prefix rANS-coded like the rest and decoded by every sequence; then (the serving policy for a prefix every
    # sequence reads each step) stored as INT8 groups inside the same pool, decoded per sequence by the batched
    # kernel and, the headline of this config, by the cascade entry point that streams it once per KV head for all
    # 256 query sets.
    runs = (("shared_prefix_rans", None, 0), ("shared_prefix_batched", {0: P // 64}, 0),
            ("shared_prefix", {0: P // 64}, P // 64))
    kvb, built_raw = None, None
    for name, raw, cascade in runs:
        if kvb is None or built_raw != raw:
            kvb = None
            kvb = kv.build_batched(kv.CODEC_RANS_HYBRID, src_a, S, H, np.full(S, T, np.uint32), D, tables, "cuda:0",
                                   keep_host=True, shared={s: (0, P // 64) for s in range(1, S)}, raw_groups=raw)
            built_raw = raw
        qp = np.full(S, T - 1, np.uint32)
        q, out, t = run(kvb, S, T, qp, cascade)
        s_chk = 7
        pages = []
        for h in range(H):
            pages += [(h, t0, k, v) for t0, k, v in decoded_pages(kvb, s_chk, h, T)]
        ref, _ = O.paged_attention_f64(q[s_chk], QH, H, D, gqa, T - 1, 0, sc, pages)
        err_a = normwise_err(out[s_chk], ref)
        assert err_a <= 1e-3, err_a
        res[name] = {"workload": "256 seqs x (8192 shared + 512 unique) tokens",
                     "prefix_codec": "int8" if raw else "rans_hybrid",
                     "entry": "cf_kv_paged_attention_cascade_async" if cascade else
                              "cf_kv_paged_attention_batched_async",
                     "tokens_per_s": S / t, "ms_per_step": t * 1e3, "unique_pool_bytes": kvb.pool_bytes,
                     "ratio_vs_bf16_logical": logical / kvb.pool_bytes,
                     "unique_gbs": kvb.pool_bytes / t / 1e9, "max_normwise_err": err_a}
    del kvb

    # (b) 4 x 131072
    S, T = 4, 131072
    seeds = rng.integers(0, 2 ** 63, size=S)

    def src_b(s):
        g = np.random.default_rng(int(seeds[s]))
        return g.standard_normal((H, T, D), dtype=np.float32), g.standard_normal((H, T, D), dtype=np.float32)

    kvb = kv.build_batched(kv.CODEC_RANS_HYBRID, src_b, S, H, np.full(S, T, np.uint32), D, tables, "cuda:0",
                           keep_host=True)
    qp = np.full(S, T - 1, np.uint32)
    q, out, t = run(kvb, S, T, qp)
    pages = [(0, t0, k, v) for t0, k, v in decoded_pages(kvb, 1, 0, T)]
    ref, _ = O.paged_attention_f64(q[1][:gqa], gqa, 1, D, gqa, T - 1, 0, sc, pages)
    err_b = normwise_err(out[1][:gqa], ref)
    assert err_b <= 1e-3, err_b
    step_bytes = kvb.pool_bytes + tables.size + S * H * (T // 64) * 4 + 2 * q.nbytes
    res["long_131k"] = {"workload": "4 seqs x 131072 tokens", "tokens_per_s": S / t, "ms_per_step": t * 1e3,
                        "pool_bytes": kvb.pool_bytes, "hbm_gbs": step_bytes / t / 1e9,
                        "roofline_frac": step_bytes / t / 1e9 / HBM_PEAK_GBS, "max_normwise_err_head0": err_b}
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="auto", choices=["auto", "kv", "kv32", "rrr", "copy", "c5", "seal",
                                                                  "nibble", "gather", "seam", "fm", "qw",
                                                                  "runtime"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--warm-s", type=float, default=3.0,
                    help="seconds of untimed back-to-back launches before the timed KV steps (0 for counter runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the hot path shards "
              f"by sequence / KV head with no exchange, so N-GPU throughput is N x the 1-GPU line", file=sys.stderr)
        return 2

    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.workload == "copy":
        cp = bench_copy(args.steps, args.warmup)
        print(json.dumps({"metric": "device-to-device copy GB/s", "value": cp["stream_copy_gbs"], "unit": "GB/s",
                          "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": cp["copy_ms"],
                          "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
                          "data": "synthetic", "config": {"workload": f"torch copy_ of {cp['copy_bytes']} B"}}))
        return 0
    if args.workload == "seal":
        print(json.dumps({"device_seal": bench_seal(args.steps, args.warmup, cpu=not args.no_cpu)}))
        return 0
    if args.workload == "c5":
        print(json.dumps({"c5": bench_c5(args.steps, args.warmup)}))
        return 0
    if args.workload == "fm":
        print(json.dumps({"c2_fm": bench_fm(args.steps, args.warmup, cpu=not args.no_cpu),
                          "cache_peaks": bench_cache_peaks()}))
        return 0
    if args.workload == "qw":
        print(json.dumps({"c3_matmul": bench_qw(args.steps, args.warmup)}))
        return 0
    if args.workload == "seam":
        print(json.dumps({"seam": bench_seam(args.steps, args.warmup),
                          "seam_c4": bench_seam_c4(min(args.steps, 10), 1)}))
        return 0
    if args.workload == "runtime":
        print(json.dumps({"attention_runtime": bench_runtime(args.steps, args.warmup)}))
        return 0
    if args.workload == "gather":
        print(json.dumps({"gather": bench_gather(args.steps, args.warmup)}))
        return 0
    if args.workload == "nibble":
        print(json.dumps({"nibble_pages": bench_nibble(args.steps, args.warmup, cpu=not args.no_cpu)}))
        return 0
    if args.workload in ("auto", "kv", "kv32"):
        kvr = bench_kv(args.steps, args.warmup, cpu=not args.no_cpu, check_seqs=0 if args.no_cpu else 8,
                       warm_s=args.warm_s, stream_peak=args.workload != "kv32")
        secondary = {k: v for k, v in kvr.items() if k not in ("roofline", "cpu_baseline", "tokens_per_s")}
        if args.workload != "kv32":
            k4 = bench_kv(min(args.steps, 50), 3, context=4096, cpu=False, check_seqs=4,
                          warm_s=min(args.warm_s, 1.0), stream_peak=False)
            from chromofold_amd import kv as _kv
            k8 = bench_kv(min(args.steps, 20), 2, cpu=False, check_seqs=2, warm_s=min(args.warm_s, 1.0),
                          stream_peak=False, codec=_kv.CODEC_INT8)
            secondary["c4_32k_int8_codec"] = {k: k8[k] for k in ("workload", "tokens_per_s", "ms_per_step", "kernel_ms",
                                                                 "bits_per_value", "max_normwise_err")}
            secondary["c4_32k_int8_codec"]["roofline_frac"] = k8["roofline"]["frac"]
            secondary["c4_4k"] = {k: k4[k] for k in ("workload", "tokens_per_s", "ms_per_step", "kernel_ms",
                                                     "bits_per_value", "max_normwise_err")}
            secondary["c4_4k"]["roofline_frac"] = k4["roofline"]["frac"]
        if args.workload == "auto":
            rrr = bench_rrr(args.steps, args.warmup, cpu=not args.no_cpu)
            secondary["wavelet_rank_mqs"] = rrr["rank_mqs"]
            secondary["wavelet_access_mqs"] = rrr["access_mqs"]
            secondary["wavelet_rank_roofline_frac"] = rrr["rank_roofline"]["frac"]
            secondary["wavelet_cpu_baseline"] = rrr.get("cpu_baseline")
            secondary["c1_rrr"] = {k: v for k, v in rrr.items() if k not in ("rank_roofline", "cpu_baseline")}
            secondary["c2_fm"] = bench_fm(min(args.steps, 20), 2, cpu=not args.no_cpu)
            secondary["c3_matmul"] = bench_qw(min(args.steps, 50), 3)
            secondary["c5_long_context"] = bench_c5(min(args.steps, 20), 2)
            secondary["device_seal"] = bench_seal(min(args.steps, 20), 2, cpu=not args.no_cpu)
            secondary["nibble_pages"] = bench_nibble(min(args.steps, 20), 2, cpu=not args.no_cpu)
            secondary["gathers"] = bench_gather(min(args.steps, 20), 2)
            secondary["seam"] = bench_seam(min(args.steps, 20), 2)
            secondary["seam_c4"] = bench_seam_c4(5, 1)
            secondary["attention_runtime"] = bench_runtime(min(args.steps, 20), 2)
            peaks = bench_cache_peaks()
            secondary["cache_peaks"] = peaks
            l2 = peaks["l2_read_gbs"]
            secondary["c1_rrr"]["rank_frac_of_l2"] = rrr["rank_roofline"]["achieved"] / l2
            for k in ("count_roofline", "locate_roofline", "lines_count_roofline", "lines_locate_roofline",
                      "rrr_count_roofline", "rrr_locate_roofline"):
                r = secondary["c2_fm"][k]
                r["frac_of_l2"] = r["achieved"] / l2
                if r["traffic_gbs"]:  # L2-miss traffic against the Infinity Cache's read rate
                    r["traffic_frac_of_mall"] = r["traffic_gbs"] / peaks["mall_read_gbs"]
            cp = bench_copy(10, 2)
            secondary["stream_copy_gbs"] = cp["stream_copy_gbs"]
            secondary["roofline_frac_of_stream_copy"] = kvr["roofline"]["achieved"] / cp["stream_copy_gbs"]
        line = {
            "metric": METRIC, "value": kvr["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": kvr["ms_per_step"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "u8 (sign-magnitude int8 -> exact f16 MFMA operands), f32 accumulate",
            "data": "synthetic (seeded N(0,1) K/V generated on the device)",
            "config": {"workload": "paged-KV decode, rANS-hybrid int8 pages, 32 seqs x 32768 ctx, 32 q / 8 kv heads, "
                                   "head_dim 128, 16-token pages, 1 layer, 1 decode token per seq"},
            "roofline": kvr["roofline"], "cpu_baseline": kvr.get("cpu_baseline"), "secondary": secondary,
        }
        print(json.dumps(line))
        return 0
    rrr = bench_rrr(args.steps, args.warmup, cpu=not args.no_cpu)
    line = {
        "metric": METRIC, "value": rrr["rank_mqs"], "unit": "Mq/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": rrr["rank_wall_ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u32", "data": "synthetic (seeded Zipf tokens)",
        "config": {"workload": "rrr-wavelet rank, 1,048,576 Zipf(1.1) tokens, vocab 32000, 1M queries"},
        "roofline": rrr["rank_roofline"], "cpu_baseline": rrr.get("cpu_baseline"),
        "secondary": {k: v for k, v in rrr.items() if k not in ("rank_roofline", "cpu_baseline")},
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
