#!/usr/bin/env python3
"""Benchmark of the KernRT HIP backend on one MI355X.

Headline (BASELINE.json `configs[1]`): greedy decode of a synthetic
SmolLM2-360M-shaped Llama with Q8_0x4 weights, KV cache pre-filled to 512
positions, one decode step = one token. Reported beside it:
  * the Q8_0 decode GEMV at SmolLM2-1.7B projection shapes, as HBM GB/s
    against the 8 TB/s peak (the `roofline` object: the dominant kernel);
  * the 128-token Q8_0 prefill at 1.7B shapes (`configs[2]`), its
    projection-kernel time and int8 ops rate against the 5.0 POPS peak;
  * the CPU baseline: the oracle's restatement of the reference cpu backend
    timed on this host on a bounded sample of the same decode.

Prints one JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
# non-packed f32 VALU lane operations per second: 256 CUs x 4 SIMDs x 16 lanes
# x 2.4 GHz. Every (row, column, block) of an exact Q8_0 GEMM costs 4 of them
# (cvt, two multiplies, add), which bounds the prefill GEMM below the MFMA peak.
VALU_LANE_OPS_PER_S = 256 * 4 * 16 * 2.4e9
METRIC = "decode tok/s + Q8_0 GEMV HBM GB/s (% peak); prefill int8 MFMA util, 1 GPU"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# SmolLM2-360M shape
CFG2 = dict(dim=960, hidden_dim=2560, n_layers=32, n_heads=15, n_kv_heads=5, vocab_size=49152, seq_len=1024,
            rms_eps=1e-5, rope_theta=100_000.0, rope_interleaved=False, head_dim=64)
# SmolLM2-1.7B shape
CFG3 = dict(dim=2048, hidden_dim=8192, n_layers=24, n_heads=32, n_kv_heads=32, vocab_size=49152, seq_len=256,
            rms_eps=1e-5, rope_theta=130_000.0, rope_interleaved=False, head_dim=64)
PREFILL_POS = 512
# LFM2-700M shape (conv layers and 6 GQA attention layers)
CFG4 = dict(dim=1536, hidden_dim=4608, n_layers=16, n_heads=24, n_kv_heads=8, vocab_size=65536, seq_len=8192,
            rms_eps=1e-5, rope_theta=1_000_000.0, rope_interleaved=False, head_dim=64)
CFG4_ATTENTION = (2, 5, 8, 10, 12, 14)
# Qwen3-0.6B shape (head_dim 128, QK-norm)
CFG5 = dict(dim=1024, hidden_dim=3072, n_layers=28, n_heads=16, n_kv_heads=8, vocab_size=151936, seq_len=2048,
            rms_eps=1e-6, rope_theta=1_000_000.0, rope_interleaved=False, head_dim=128)


def synthetic_model(K, cfg: dict, storage: str, seed: int, qk_norm: bool = False, lfm2_attention=None):
    """Device-generated N(0, 0.02) Q8 weights (tied classifier), unit norms.
    With `lfm2_attention` (the attention layer indices) an LFM2 hybrid: the
    other layers are short convolutions (kernel 3, weights N(0, 0.02))."""
    hip = K.open("hip")
    c = K.Config(**cfg)
    layers, handles = [], []
    s = seed
    rng = np.random.default_rng(seed)
    ones = np.ones(c.dim, np.float32)
    for l in range(c.n_layers):
        attention = lfm2_attention is None or l in lfm2_attention
        if attention:
            shapes = {"q": (c.q_dim, c.dim), "k": (c.kv_dim, c.dim), "v": (c.kv_dim, c.dim), "o": (c.dim, c.q_dim)}
        else:
            shapes = {"conv_in": (3 * c.dim, c.dim), "conv_out": (c.dim, c.dim)}
        shapes.update({"gate": (c.hidden_dim, c.dim), "up": (c.hidden_dim, c.dim), "down": (c.dim, c.hidden_dim)})
        h = {}
        for name, (n, k) in shapes.items():
            s += 1
            h[name] = hip.synthetic_matrix(storage, n, k, s)
        handles.append(h)
        qk = np.ones(c.head_dim, np.float32) if (qk_norm and attention) else None
        conv = None if attention else (rng.standard_normal((c.dim, 3), dtype=np.float32) * np.float32(0.02))
        layers.append(K.LayerWeights(ones, ones, rms_q=qk, rms_k=qk, conv_kernel=conv, is_attention=attention))
    emb = hip.synthetic_matrix(storage, c.vocab_size, c.dim, seed + 100_000)
    hip.bind_handles(emb, 0xFFFFFFFF, handles)
    model = K.Model(c, hip, None, lfm2=lfm2_attention is not None, layers=layers, rms_final=ones)
    model.weight_handles = (emb, handles)  # for checkers that read the device bytes back
    return hip, model, c


def bench_decode(K, steps: int, warmup: int, use_graph: bool = True):
    log("decode: building the 360M-shaped Q8_0x4 model on the device")
    hip, model, c = synthetic_model(K, CFG2, "q8_0x4", seed=2)
    hip.kv_synthetic(PREFILL_POS, seed=5)
    token0 = int(np.random.default_rng(2).integers(0, c.vocab_size))
    hip.synchronize()
    log(f"decode: warmup {warmup} tokens (captures the step graph)")
    model.generate_greedy(token0, PREFILL_POS, max(warmup, 1), use_graph=use_graph)
    hip.synchronize()
    log(f"decode: timing {steps} greedy tokens from position {PREFILL_POS}")
    t0 = time.perf_counter()
    toks = model.generate_greedy(token0, PREFILL_POS, steps, use_graph=use_graph)
    hip.synchronize()
    dt = time.perf_counter() - t0
    # the per-call forward() path (logits back to the host each call) with
    # the reference's decode_rate method (examples/decode_rate.rs:62-79): 5
    # warm-up calls, then 300 timed calls of one token at one position; p10
    # and median
    for _ in range(5):
        model.forward(token0, PREFILL_POS)
    samples = []
    for _ in range(300):
        t1 = time.perf_counter()
        model.forward(token0, PREFILL_POS)
        samples.append(time.perf_counter() - t1)
    samples.sort()
    fwd_p10, fwd_med = samples[len(samples) // 10], samples[len(samples) // 2]
    weights = sum(n * k for n, k in [(c.q_dim, c.dim), (c.kv_dim, c.dim), (c.kv_dim, c.dim), (c.dim, c.q_dim),
                                     (c.hidden_dim, c.dim), (c.hidden_dim, c.dim),
                                     (c.dim, c.hidden_dim)]) * c.n_layers + c.vocab_size * c.dim
    p_mean = PREFILL_POS + steps / 2
    kv_bytes = 2 * c.n_layers * (p_mean + 1) * c.kv_dim * 4
    bytes_tok = weights * (1 + 2 / 32) + kv_bytes  # int8 + f16 scales per 32-block
    out = dict(tok_s=steps / dt, ms_per_tok=dt * 1e3 / steps, forward_tok_s=1.0 / fwd_med,
               forward_p10_tok_s=1.0 / fwd_p10, forward_samples=len(samples),
               bytes_per_token=bytes_tok, hbm_gbs_per_token_model=bytes_tok * steps / dt / 1e9,
               first_tokens=[int(t) for t in toks[:8]])
    model.close()
    hip.close()
    return out


def gemv_algo_bytes(n: int, k: int) -> int:
    """Algorithmic HBM bytes of one Q8_0 GEMV launch over n weight rows of
    in_dim k at M = 1: int8 weights, f32 block scales, the quantized
    activation row with its f32 scales, and the f32 outputs."""
    nb = k // 32
    return n * k + n * nb * 4 + k + nb * 4 + n * 4


def read_sweep(hip, big, big_n: int, sizes: dict, passes: int = 3):
    """The bare streaming read (kr_stream_read_shape) of each launch size in
    every shape: 1, 2, 4 or 8 16-byte loads per lane per round, one round
    per workgroup or 256..2048 workgroups looping. Each size is read from
    distinct offsets of a 2 GiB buffer, over 2x the 256 MB MALL per pass, so
    the reads are cold as the decode pass's are; a pass is captured and
    replayed like the GEMV's."""
    out = {}
    for key, b in sizes.items():
        n4 = ((b + 15) // 16) * 4
        launches = max(24, -(-(512 << 20) // (4 * n4)))
        offs = [(i * n4) % (big_n - n4) // 4 * 4 for i in range(launches)]
        rows = []
        for cpl in (1, 2, 4, 8):
            full = -(-n4 // (4 * 256 * cpl))
            for wgs in (0, 256, 512, 1024, 2048):
                if wgs >= full:
                    continue
                hip.capture_begin()
                for off in offs:
                    hip.stream_read(big, off, n4, cpl, wgs)
                hip.capture_end()
                hip.replay(1)
                hip.synchronize()
                hip.replay(1)
                hip.timer_start()
                hip.replay(passes)
                us = hip.timer_stop() * 1e3 / (passes * launches)
                rows.append(dict(chunks_per_lane=cpl, workgroups=wgs or full, us=round(us, 3),
                                 gbs=round(4 * n4 / (us * 1e-6) / 1e9, 1)))
        best = min(rows, key=lambda r: r["us"])
        out[key] = dict(bytes=b, launches_per_pass=launches, best=best, shapes=rows)
    return out


def bench_gemv(K, reps: int = 3, use_graph: bool = True):
    """Q8_0 decode GEMVs (M = 1) at SmolLM2-1.7B shapes, launched as a decode
    step launches them: per layer the fused QKV (3 x 2048x2048, one launch),
    O 2048x2048, the fused gate+up (2 x 8192x2048, one launch) and down
    2048x8192, over 24 layers of distinct weights, plus the 49152x2048
    classifier. One pass streams 1.93 GB of weights, far beyond the 256 MB
    MALL, so every launch reads its weights from HBM. Launches are grouped by
    in_dim (the activation workspace holds one quantized row): first every
    in_dim-2048 launch of all layers, then every down projection."""
    log("gemv: building 24 layers of 1.7B-shaped Q8_0 matrices")
    hip = K.open("hip")
    c = K.Config(**CFG3)
    d, hdim = c.dim, c.hidden_dim
    seed = 1000
    layers = []
    for l in range(c.n_layers):
        m = {}
        for name, (n, k) in {"q": (d, d), "k": (d, d), "v": (d, d), "o": (d, d), "gate": (hdim, d),
                             "up": (hdim, d), "down": (d, hdim)}.items():
            seed += 1
            m[name] = hip.synthetic_matrix("q8_0", n, k, seed)
        layers.append(m)
    cls = hip.synthetic_matrix("q8_0", c.vocab_size, d, 99)
    rng = np.random.default_rng(3)
    x_d = hip.upload(rng.normal(size=d).astype(np.float32))
    x_h = hip.upload(rng.normal(size=hdim).astype(np.float32))
    y = {n: [hip.alloc(n) for _ in range(3)] for n in (d, hdim, c.vocab_size)}
    # (matrices, out rows per matrix, in_dim) per launch, in launch order
    group_a = []
    for m in layers:
        group_a += [([m["q"], m["k"], m["v"]], d, d), ([m["o"]], d, d), ([m["gate"], m["up"]], hdim, d)]
    group_a.append(([cls], c.vocab_size, d))
    group_b = [([m["down"]], d, hdim) for m in layers]

    # launch arguments prepared once: the host must issue launches faster than
    # the GPU retires them, or the events would time the host
    import ctypes as C
    fn, ctx = hip._L.kr_matmul_quantized_set, hip.ctx
    prepared = {}
    for g in group_a + group_b:
        mats, n, _ = g
        prepared[id(g)] = ((C.c_uint32 * len(mats))(*mats), (C.c_uint32 * len(mats))(*y[n][:len(mats)]), len(mats))

    def run(group):
        for g in group:
            ws, ys, nm = prepared[id(g)]
            if fn(ctx, ws, ys, nm, 1) != 0:
                raise RuntimeError(hip._L.kr_last_error(ctx).decode())

    # Without graphs (for profilers) the launches are issued one by one from
    # here, slower than the GPU retires them; an MFMA spin of a few ms ahead
    # of them keeps the GPU busy while they queue, so they then run back to
    # back as a graph replay runs them (not each after an idle gap).
    hip.mfma_rate(0, 256, 100)
    hip.synchronize()
    hip.timer_start()
    hip.mfma_rate(0, 256, 2000)
    spin_iters_per_ms = 2000 / hip.timer_stop()

    def timed(group, passes):
        """One pass captured into a HIP graph, as the decode driver replays its
        step; the graph is then replayed `passes` times between two events.
        Without graphs the launches are issued directly behind a spin."""
        run(group)  # warm-up pass (also evicts the other group from the MALL)
        if not use_graph:
            hip.synchronize()
            hip.mfma_rate(0, 256, max(1, int(spin_iters_per_ms * 0.03 * passes * len(group))))
            hip.timer_start()
            for _ in range(passes):
                run(group)
            return hip.timer_stop()
        hip.capture_begin()
        run(group)
        hip.capture_end()
        hip.replay(1)
        hip.synchronize()
        hip.replay(1)  # keeps the GPU busy while the timed launches are submitted
        hip.timer_start()
        hip.replay(passes)
        return hip.timer_stop()

    kinds = {}
    total_ms, total_bytes, total_launches = 0.0, 0, 0
    for x, width, group in ((x_d, d, group_a), (x_h, hdim, group_b)):
        hip.quantize_rows(x, 1, width)
        ms = timed(group, reps)
        total_ms += ms
        total_launches += reps * len(group)
        for mats, n, k in group:
            total_bytes += reps * gemv_algo_bytes(n * len(mats), k)
            kinds.setdefault(f"{len(mats)}x{n}x{k}", [0, gemv_algo_bytes(n * len(mats), k)])[0] += 1
    gbs = total_bytes / (total_ms * 1e-3) / 1e9
    # the practical ceiling: a bare streaming read of each launch's bytes, in
    # the same order and from a 2 GiB rotation (cold), timed the same way
    big_n = 512 << 20
    big = hip.alloc(big_n)
    read_sizes = [((gemv_algo_bytes(n * len(mats), k) + 15) // 16) * 4 for mats, n, k in group_a + group_b]
    offs, o = [], 0
    for n4 in read_sizes:
        if o + n4 > big_n:
            o = 0
        offs.append(o)
        o += n4

    def reads():
        for off, n4 in zip(offs, read_sizes):
            hip.stream_read(big, off, n4)

    reads()
    if use_graph:
        hip.capture_begin()
        reads()
        hip.capture_end()
        hip.replay(1)
        hip.synchronize()
        hip.replay(1)
        hip.timer_start()
        hip.replay(reps)
    else:
        hip.synchronize()
        hip.mfma_rate(0, 256, max(1, int(spin_iters_per_ms * 0.03 * reps * len(read_sizes))))
        hip.timer_start()
        for _ in range(reps):
            reads()
    read_ms = hip.timer_stop()
    read_gbs = sum(read_sizes) * 4 * reps / (read_ms * 1e-3) / 1e9
    sweep = read_sweep(hip, big, big_n, {key: b for key, (_, b) in kinds.items()}) if use_graph else None
    # per launch shape: time each kind alone over the same distinct matrices
    per_shape = {}
    for key, (count, b) in kinds.items():
        nm, n, k = (int(t) for t in key.split("x"))
        group = [g for g in group_a + group_b if len(g[0]) == nm and g[1] == n and g[2] == k]
        hip.quantize_rows(x_d if k == d else x_h, 1, k)
        us = timed(group, 4) * 1e3 / (4 * len(group))
        per_shape[key] = dict(launches_per_pass=count, bytes=b, avg_us=round(us, 3),
                              gbs=round(b / (us * 1e-6) / 1e9, 1))
    # one GEMV at SmolLM2-135M's gate shape,
    # 1536x576. The kernel alone, over 512 distinct copies of the matrix
    # (512 MB, twice the MALL, so each launch reads HBM), the activation
    # quantized once beforehand, one pass captured in a graph and replayed.
    n_cfg1 = 512
    m1 = [hip.synthetic_matrix("q8_0", 1536, 576, 7700 + i) for i in range(n_cfg1)]
    x1 = hip.upload(rng.normal(size=576).astype(np.float32))
    y1 = [hip.alloc(1536)]
    g1 = [([m], 1536, 576) for m in m1]
    for g in g1:
        prepared[id(g)] = ((C.c_uint32 * 1)(g[0][0]), (C.c_uint32 * 1)(*y1), 1)
    hip.quantize_rows(x1, 1, 576)
    cfg1_us = timed(g1, 4) * 1e3 / (4 * n_cfg1)
    # and as a caller sees one projection: quantize + GEMV issued eagerly,
    # on one cache-resident matrix
    for _ in range(10):
        hip.matmul(m1[0], x1, y1[0], 1)
    hip.synchronize()
    hip.timer_start()
    for _ in range(200):
        hip.matmul(m1[0], x1, y1[0], 1)
    cfg1_call_us = hip.timer_stop() * 1e3 / 200
    # a plain 64 MiB device copy (k_copy): the reference for scaling the HBM
    # byte counters of a profiler run, and a practical streaming rate
    n_copy = 16 << 20
    src, dst = hip.alloc(n_copy), hip.alloc(n_copy)
    hip.copy(src, 0, dst, 0, n_copy)
    hip.synchronize()
    hip.timer_start()
    for _ in range(10):
        hip.copy(src, 0, dst, 0, n_copy)
    copy_us = hip.timer_stop() * 1e3 / 10
    hip.close()
    swept = None
    if sweep:
        # the pass read at each launch size's best shape: the ceiling the
        # GEMV's launch sizes allow a read-only kernel
        t_best = sum(cnt * sweep[key]["best"]["us"] for key, (cnt, _) in kinds.items())
        swept = dict(gbs=round(sum(cnt * b for cnt, b in kinds.values()) / (t_best * 1e-6) / 1e9, 1),
                     us_per_launch=round(t_best / sum(cnt for cnt, _ in kinds.values()), 3),
                     per_size={key: v["best"] for key, v in sweep.items()})
    return dict(achieved_gbs=gbs, avg_launch_us=total_ms * 1e3 / total_launches,
                read_ceiling_gbs=read_gbs, read_ceiling_us_per_launch=read_ms * 1e3 / total_launches,
                swept_read_ceiling=swept, read_sweep=sweep,
                bytes_per_launch=total_bytes / total_launches, launches_per_pass=len(group_a) + len(group_b),
                bytes_per_pass=total_bytes // reps, per_shape=per_shape,
                cfg1_1536x576_us=cfg1_us, cfg1_bytes=1_003_776,
                cfg1_gbs=gemv_algo_bytes(1536, 576) / (cfg1_us * 1e-6) / 1e9,
                cfg1_rotated_copies=n_cfg1, cfg1_eager_matmul_us=cfg1_call_us,
                copy_64mib_us=copy_us, copy_gbs=2 * 4 * n_copy / (copy_us * 1e-6) / 1e9)


def bench_prefill(K, reps: int = 2):
    """128-token Q8_0 prefill at 1.7B projection shapes (`configs[2]`): the
    int8 MFMA GEMM launches the model's prefill issues per layer -- fused
    q/k/v (one launch over 6144 rows), o, fused gate/up (16384 rows), down in
    its chain-split form (four partial-sum planes, kr_matmul_split) -- alone
    (activations quantized beforehand), and the projections with their
    activation quantization, over all 24 layers' distinct matrices. The
    planes' sum runs in the norm launch that follows down in the model."""
    log("prefill: 128-row Q8_0 projections at 1.7B shapes")
    hip = K.open("hip")
    c = K.Config(**CFG3)
    m_rows = 128
    groups = [("qkv", [(c.q_dim, c.dim), (c.kv_dim, c.dim), (c.kv_dim, c.dim)]), ("o", [(c.dim, c.q_dim)]),
              ("gate_up", [(c.hidden_dim, c.dim), (c.hidden_dim, c.dim)]), ("down", [(c.dim, c.hidden_dim)])]
    mats = [[[hip.synthetic_matrix("q8_0", n, k, 5000 * l + 10 * g + i) for i, (n, k) in enumerate(shapes)]
             for g, (_, shapes) in enumerate(groups)] for l in range(c.n_layers)]
    rng = np.random.default_rng(4)
    ks = {k for _, shapes in groups for _, k in shapes}
    xs = {k: hip.upload(rng.normal(size=m_rows * k).astype(np.float32)) for k in ks}
    split = [name == "down" for name, _ in groups]  # the model's chain-split launch
    ys = [[hip.alloc((4 if split[g] else 1) * m_rows * n) for n, _ in shapes] for g, (_, shapes) in enumerate(groups)]

    def launch(l, g, quantize):
        k = groups[g][1][0][1]
        if split[g]:
            hip.matmul_split(mats[l][g][0], xs[k] if quantize else None, ys[g][0], m_rows)
        else:
            if quantize:
                hip.quantize_rows(xs[k], m_rows, k)
            hip.matmul_quantized_set(mats[l][g], ys[g], m_rows)

    def run():
        for l in range(c.n_layers):
            for g in range(len(groups)):
                launch(l, g, True)

    run()
    hip.synchronize()
    hip.timer_start()
    run()
    proj_ms = hip.timer_stop()
    # GEMM kernels only: one launch group at a time over the 24 layers' matrices
    gemm_ms, per_shape = 0.0, {}
    for g, (name, shapes) in enumerate(groups):
        k = shapes[0][1]
        n = sum(nn for nn, _ in shapes)
        launch(0, g, True)
        for l in range(c.n_layers):
            launch(l, g, False)
        hip.synchronize()
        hip.timer_start()
        for _ in range(reps):
            for l in range(c.n_layers):
                launch(l, g, False)
        ms = hip.timer_stop() / reps
        gemm_ms += ms
        us = ms * 1e3 / c.n_layers
        valu_floor_us = m_rows * n * (k // 32) * 4 / VALU_LANE_OPS_PER_S * 1e6
        per_shape[f"{name} {n}x{k}"] = dict(avg_us=us, tops=2 * m_rows * n * k / (us * 1e-6) / 1e12,
                                           weight_gbs=n * k * (1 + 4 / 32) / (us * 1e-6) / 1e9,
                                           valu_floor_us=valu_floor_us, frac_of_valu_floor=valu_floor_us / us,
                                           valu_floor_3op_us=valu_floor_us * 3 / 4,
                                           frac_of_valu_floor_3op=valu_floor_us * 3 / 4 / us)
    ops = 2 * m_rows * sum(n * k for _, shapes in groups for n, k in shapes) * c.n_layers
    tops = ops / (gemm_ms * 1e-3) / 1e12
    triples = m_rows * sum(n * k // 32 for _, shapes in groups for n, k in shapes) * c.n_layers
    valu_floor_ms = triples * 4 / VALU_LANE_OPS_PER_S * 1e3
    hip.close()
    # valu_floor: the exact epilogue's 4 vector operations per (row, column,
    # block) -- cvt, two multiplies, add; valu_floor_3op: 3, with the scale
    # product sa * sb on the matrix core as the wide tiles do
    return dict(rows=m_rows, gemm_ms=gemm_ms, int8_tops=tops, mfma_util=tops / INT8_PEAK_TOPS, ops=ops,
                valu_floor_ms=valu_floor_ms, frac_of_valu_floor=valu_floor_ms / gemm_ms,
                valu_floor_3op_ms=valu_floor_ms * 3 / 4, frac_of_valu_floor_3op=valu_floor_ms * 3 / 4 / gemm_ms,
                projection_ms_with_quantize=proj_ms, per_shape=per_shape)


def bench_mfma_peak(K, workgroups: int = 2048, iters: int = 20000):
    """The chip's dense int8 MFMA rate measured with a probe kernel (four
    independent MFMAs in flight per wave, 8 workgroups of 4 waves per CU),
    for the 32x32x32 instruction and for the 16x16x32 one the Q8_0 GEMM
    issues -- the measured counterpart of the vendor's 5.0 POPS."""
    hip = K.open("hip")
    out = {}
    for kind, name in ((0, "i32_32x32x32_i8"), (1, "i32_16x16x32_i8")):
        hip.mfma_rate(kind, workgroups, 100)
        hip.synchronize()
        hip.timer_start()
        ops = hip.mfma_rate(kind, workgroups, iters)
        ms = hip.timer_stop()
        out[name] = dict(tops=ops / (ms * 1e-3) / 1e12, ms=ms)
    hip.close()
    return out


def prefill_rate(model, toks, reps: int = 20):
    """The reference's prefill_rate method (examples/prefill_rate.rs:98-119):
    the first call timed on its own, then `reps` calls; best and median.
    Each call reads its logits back, so it ends with the device idle."""
    t0 = time.perf_counter()
    model.prefill(toks, 0)
    first = time.perf_counter() - t0
    samples = []
    for _ in range(reps):
        t0 = time.perf_counter()
        model.prefill(toks, 0)
        samples.append(time.perf_counter() - t0)
    samples.sort()
    best, median = samples[0], samples[len(samples) // 2]
    n = len(toks)
    return dict(tokens=n, tok_s=n / best, median_tok_s=n / median, best_ms=best * 1e3, median_ms=median * 1e3,
                first_call_ms=first * 1e3, calls=reps)


def bench_prefill_model(K, n_tokens: int = 128):
    """`configs[2]` end to end: a 128-token prefill of the synthetic
    SmolLM2-1.7B-shaped Llama with Q8_0 weights, seeded random token ids."""
    log("prefill model: building the 1.7B-shaped Q8_0 model on the device")
    hip, model, c = synthetic_model(K, CFG3, "q8_0", seed=7)
    toks = [int(t) for t in np.random.default_rng(8).integers(0, c.vocab_size, size=n_tokens)]
    out = prefill_rate(model, toks)
    model.close()
    hip.close()
    return out


def bench_cfg4(K, n_prompt: int = 128, n_decode: int = 256, use_graph: bool = True):
    """`configs[3]`: the LFM2-700M-shaped hybrid with Q8_0x4 weights, a
    128-token prefill of seeded random ids, then 256 greedy decode tokens
    (context cap 8192), the decode replaying the captured step graph."""
    log("cfg4: building the LFM2-700M-shaped Q8_0x4 hybrid on the device")
    hip, model, c = synthetic_model(K, CFG4, "q8_0x4", seed=11, qk_norm=True, lfm2_attention=CFG4_ATTENTION)
    toks = [int(t) for t in np.random.default_rng(12).integers(0, c.vocab_size, size=n_prompt)]
    pre = prefill_rate(model, toks)
    first = int(np.argmax(model.prefill(toks, 0)))
    model.generate_greedy(first, n_prompt, 8, use_graph=use_graph)
    hip.synchronize()
    t0 = time.perf_counter()
    model.generate_greedy(first, n_prompt, n_decode, use_graph=use_graph)
    hip.synchronize()
    decode_s = time.perf_counter() - t0
    model.close()
    hip.close()
    return dict(prefill_tokens=n_prompt, prefill_tok_s=pre["tok_s"], prefill_median_tok_s=pre["median_tok_s"],
                prefill_first_ms=pre["first_call_ms"], decode_tokens=n_decode, decode_tok_s=n_decode / decode_s)


def bench_cfg5(K, n_prompt: int = 2048, n_seq: int = 64, ctx: int = 1024, steps: int = 8):
    """`configs[4]`: the Qwen3-0.6B-shaped Llama (head_dim 128, QK-norm) with
    Q8_0 weights. (i) a 2048-token prefill of seeded random ids (best and
    median of 20 after a timed first call); (ii) batched decode of 64 sequences, each with
    a 1024-position KV cache of its own (N(0, 1), 64 x 1024 slots in one
    cache): every step is one row per sequence, so every projection and the
    151936x1024 lm_head run as M = 64 int8 GEMMs; logits stay on the device."""
    log("cfg5: building the Qwen3-0.6B-shaped Q8_0 model (prefill)")
    hip, model, c = synthetic_model(K, CFG5, "q8_0", seed=21, qk_norm=True)
    toks = [int(t) for t in np.random.default_rng(22).integers(0, c.vocab_size, size=n_prompt)]
    pre = prefill_rate(model, toks)
    best, first = pre["best_ms"] * 1e-3, pre["first_call_ms"] * 1e-3
    model.close()
    hip.close()
    log("cfg5: batched decode, 64 sequences x 1024-position caches")
    cfg = dict(CFG5, seq_len=n_seq * ctx)
    hip, model, c = synthetic_model(K, cfg, "q8_0", seed=23, qk_norm=True)
    hip.kv_synthetic(n_seq * ctx, seed=24)
    rng = np.random.default_rng(25)
    tok = [int(t) for t in rng.integers(0, c.vocab_size, size=n_seq)]
    pos = [ctx - 1] * n_seq
    slots = [s * ctx + ctx - 1 for s in range(n_seq)]
    starts = [s * ctx for s in range(n_seq)]
    model.decode_batch(tok, pos, slots, starts, read=False)
    hip.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.decode_batch(tok, pos, slots, starts, read=False)
    hip.synchronize()
    dt = time.perf_counter() - t0
    kv_bytes = 2 * c.n_layers * n_seq * ctx * c.kv_dim * 4
    model.close()
    hip.close()
    return dict(prefill_tokens=n_prompt, prefill_tok_s=n_prompt / best, prefill_best_ms=best * 1e3,
                prefill_median_ms=pre["median_ms"], prefill_first_ms=first * 1e3, batch_sequences=n_seq,
                batch_ctx=ctx,
                batch_step_ms=dt * 1e3 / steps, batch_tok_s=n_seq * steps / dt,
                batch_kv_gbs=kv_bytes * steps / dt / 1e9)


def host_cpu():
    """The host CPU model name and the cores this process may use."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return name, os.cpu_count(), usable


def cpu_decode_leg(K, budget: float, max_steps: int = 300):
    """The oracle's cpu backend decoding the decode leg's model on one core:
    the synthetic weights and the pre-filled cache are generated on the
    device with the decode leg's seeds and read back, so both sides hold the
    same bytes. A GPU greedy run of `max_steps` tokens from the same start is
    the reference sequence: every CPU token is compared with it. Each CPU
    greedy step is one tg1 sample; p10 and median as the reference's
    decode_rate reports (examples/decode_rate.rs:62-79), over the steps that
    fit `budget` seconds (at most `max_steps`)."""
    import oracle as O
    cpu_name, n_cpu, usable = host_cpu()
    log(f"cpu baseline ({O.VARIANT or 'o2'} oracle): reading the decode leg's weights and cache back")
    hip, model, c = synthetic_model(K, CFG2, "q8_0x4", seed=2)
    hip.kv_synthetic(PREFILL_POS, seed=5)
    token0 = int(np.random.default_rng(2).integers(0, c.vocab_size))
    gpu_tokens = [int(t) for t in model.generate_greedy(token0, PREFILL_POS, max_steps, use_graph=True)]
    emb, handles = model.weight_handles
    oc = O.Config(**CFG2)
    w = O.Weights(c.n_layers)

    def omat(h):
        _, n, k = hip.matrix_shape(h)
        q, sc = hip.read_matrix(h)
        return O.Matrix.from_q8_0x4_blocks(K.backends.q8_0x4_records(q, sc), n, k)

    for l in range(c.n_layers):
        for name, h in handles[l].items():
            w.set_proj(l, name, omat(h))
        w.set_norm(l, "att", np.ones(c.dim, np.float32))
        w.set_norm(l, "ffn", np.ones(c.dim, np.float32))
    w.set_embedding(omat(emb))
    w.set_final_norm(np.ones(c.dim, np.float32))
    w.set_classifier(None)
    cpu = O.Model(oc, w, "cpu")
    per = PREFILL_POS * c.kv_dim
    for l in range(c.n_layers):
        for which in (0, 1):
            cpu.kv_upload(which, l * c.seq_len * c.kv_dim, hip.kv_read(which, l * c.seq_len * c.kv_dim, per))
    model.close()
    hip.close()
    log(f"cpu baseline ({O.VARIANT or 'o2'} oracle): timing greedy decode steps on one core")
    tok, toks, times, t0 = token0, [], [], time.perf_counter()
    while len(times) < max_steps and time.perf_counter() - t0 < budget:
        s0 = time.perf_counter()
        logits = cpu.forward(tok, PREFILL_POS + len(times))
        times.append(time.perf_counter() - s0)
        tok = O.argmax(logits)
        toks.append(tok)
    del cpu, w
    st = sorted(times)
    median, p10 = st[len(st) // 2], st[len(st) // 10]
    return dict(median_s=median, p10_s=p10, steps=len(times), tokens=toks, tokens_compared=len(toks),
                all_tokens_match_gpu=toks == gpu_tokens[:len(toks)], host_cpu=cpu_name, nproc=n_cpu,
                cores_usable=usable)


def bench_cpu_baseline(K, decode_budget: float = 30.0, prefill_budget: float = 15.0, max_steps: int = 300,
                       o3=None):
    """The oracle's cpu backend -- a C++ restatement of the reference's x86
    path (Q8_0x4: quantize_rows + gemm_q8_0x4_batched, re-quantizing logits;
    Q8_0: per-row quantize + dot_q8_0_scalar), built -O2 -ffp-contract=off,
    on 1 core, on the very bytes the GPU legs use.

    decode: cpu_decode_leg. `o3` is the same leg run on the -O3
    build of the oracle (the same bits, labelled as this build's variant),
    measured in a child process before this one touched the GPU.
    prefill: one layer's seven Q8_0 projections at 128 rows
    (layer 0 of the prefill leg's weights), the first call timed apart and
    the best of the repeats that fit `prefill_budget`
    (examples/prefill_rate.rs:98-119), scaled to the 24-layer model."""
    import oracle as O
    dec = cpu_decode_leg(K, decode_budget, max_steps)
    median, p10, cpu_name, n_cpu, usable = dec["median_s"], dec["p10_s"], dec["host_cpu"], dec["nproc"], \
        dec["cores_usable"]
    log("cpu baseline: one 1.7B layer's prefill projections on one core")
    hip, pm, c3 = synthetic_model(K, CFG3, "q8_0", seed=7)
    _, handles3 = pm.weight_handles
    shapes3 = {"q": (c3.q_dim, c3.dim), "k": (c3.kv_dim, c3.dim), "v": (c3.kv_dim, c3.dim),
               "o": (c3.dim, c3.q_dim), "gate": (c3.hidden_dim, c3.dim), "up": (c3.hidden_dim, c3.dim),
               "down": (c3.dim, c3.hidden_dim)}
    mats = {}
    for name, (n, k) in shapes3.items():
        q, sc = hip.read_matrix(handles3[0][name], "q8_0", n, k)
        mats[name] = O.Matrix.from_q8_0(q.ravel(), sc.ravel(), n, k)
    pm.close()
    hip.close()
    rng = np.random.default_rng(12)
    xs = {k: rng.normal(size=(128, k)).astype(np.float32) for k in (c3.dim, c3.hidden_dim)}

    def layer():
        s0 = time.perf_counter()
        for name, (n, k) in shapes3.items():
            mats[name].project_cpu(xs[k])
        return time.perf_counter() - s0

    first = layer()
    reps, t1 = [], time.perf_counter()
    while len(reps) < 20 and time.perf_counter() - t1 + first < prefill_budget:
        reps.append(layer())
    best = min(reps) if reps else first
    ops = 2 * 128 * sum(n * k for n, k in shapes3.values())
    prefill = dict(tokens=128, layer_first_s=first, layer_best_s=best, layer_repeats=len(reps),
                   tok_s_24_layers=128 / (best * c3.n_layers), gops=ops / best / 1e9)
    out = dict(value=1.0 / median, unit="tok/s", cores=1, kind="port",
               sample=f"{dec['steps']} greedy decode steps of the cfg2 360M-shaped Q8_0x4 model (the decode leg's "
                      f"device-generated weights and cache, read back) from position {PREFILL_POS}, oracle cpu "
                      f"backend (scalar C++ port of the reference's x86 path, g++ -O2 -ffp-contract=off), "
                      f"1 thread on {cpu_name} ({usable} of {n_cpu} cores usable); median step "
                      f"{median * 1e3:.1f} ms, p10 {p10 * 1e3:.1f} ms; every token compared with a GPU greedy run",
               host_cpu=cpu_name, nproc=n_cpu, cores_usable=usable, p10_tok_s=1.0 / p10,
               median_ms=median * 1e3, steps=dec["steps"], first_tokens=dec["tokens"][:8],
               all_tokens_match_gpu=dec["all_tokens_match_gpu"], tokens_compared=dec["tokens_compared"],
               prefill=prefill)
    if o3:
        out["o3_variant"] = dict(
            label="this build's variant: the same oracle at g++ -O3 -ffp-contract=off (no fast-math; "
                  "the same bits), 1 thread",
            tok_s=1.0 / o3["median_s"], p10_tok_s=1.0 / o3["p10_s"], median_ms=o3["median_s"] * 1e3,
            steps=o3["steps"], all_tokens_match_gpu=o3["all_tokens_match_gpu"],
            tokens_compared=o3["tokens_compared"])
    return out


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "k_gemv_q8_0_1p7b_decode_pmc.md")


def measured_traffic():
    """HBM bytes per GEMV launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE runs of `bench.py --only gemv`, scaled by the
    same counters on a 64 MiB copy); None if the summary is absent."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch"):
                    return float(line.split("=")[1])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only", choices=["decode", "gemv", "prefill", "cfg4", "cfg5", "cpu", "cpu-decode-leg"],
                    default=None)
    ap.add_argument("--cpu-budget", type=float, default=30.0,
                    help="seconds of CPU decode steps per oracle build (at most --cpu-steps; the reference's "
                         "decode_rate takes 300)")
    ap.add_argument("--cpu-steps", type=int, default=300)
    ap.add_argument("--no-o3", action="store_true", help="skip the -O3 oracle figure")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the decode step's and the GEMV passes' kernels directly instead of replaying "
                         "captured HIP graphs (same kernels; for profilers that cannot trace graph launches)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every projection would "
              "shard by output rows, with an all-gather of the f32 input rows in front of O and down, so that "
              "each output's f32 chain stays on one GPU).", file=sys.stderr)
        sys.exit(2)
    if args.only == "cpu-decode-leg":
        # child mode: one oracle build's decode leg, JSON on stdout
        import kernrt_amd as K
        dec = cpu_decode_leg(K, args.cpu_budget, args.cpu_steps)
        dec.pop("tokens")
        print(json.dumps(dec), flush=True)
        return
    want_cpu = not args.skip_cpu and args.only in (None, "cpu")
    o3 = None
    if want_cpu and not args.no_o3:
        # the -O3 oracle's decode leg runs in a child process started before
        # this process touches the GPU (the oracle library is chosen at load)
        import subprocess
        log("cpu baseline: the -O3 oracle's decode leg in a child process")
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--only", "cpu-decode-leg", "--cpu-budget",
                            str(args.cpu_budget), "--cpu-steps", str(args.cpu_steps)],
                           env=dict(os.environ, KERNRT_ORACLE_VARIANT="o3"), stdout=subprocess.PIPE, text=True)
        if r.returncode == 0:
            o3 = json.loads(r.stdout.strip().splitlines()[-1])
        else:
            log(f"cpu baseline: the -O3 leg failed ({r.returncode})")
    import kernrt_amd as K

    res = {}
    if args.only in (None, "decode"):
        res["decode"] = bench_decode(K, args.steps, args.warmup, use_graph=not args.no_graph)
        log(f"decode: {res['decode']['tok_s']:.1f} tok/s")
    if args.only in (None, "gemv"):
        res["gemv"] = bench_gemv(K, use_graph=not args.no_graph)
        log(f"gemv: {res['gemv']['achieved_gbs']:.0f} GB/s")
    if args.only in (None, "prefill"):
        res["prefill"] = bench_prefill(K)
        log(f"prefill: {res['prefill']['int8_tops']:.1f} TOPS in the GEMM kernels")
        res["prefill"]["mfma_peak_measured"] = bench_mfma_peak(K)
        res["prefill"]["model"] = bench_prefill_model(K)
        log(f"prefill model: {res['prefill']['model']['tok_s']:.0f} tok/s")
    if args.only in (None, "cfg4"):
        res["cfg4"] = bench_cfg4(K, use_graph=not args.no_graph)
        log(f"cfg4: prefill {res['cfg4']['prefill_tok_s']:.0f} tok/s, decode {res['cfg4']['decode_tok_s']:.1f} tok/s")
    if args.only in (None, "cfg5"):
        res["cfg5"] = bench_cfg5(K)
        log(f"cfg5: prefill {res['cfg5']['prefill_tok_s']:.0f} tok/s, batched decode "
            f"{res['cfg5']['batch_tok_s']:.0f} tok/s")
    if not want_cpu:
        cpu = None
    else:
        cpu = bench_cpu_baseline(K, decode_budget=args.cpu_budget, max_steps=args.cpu_steps, o3=o3)
        log(f"cpu baseline: {cpu['value']:.2f} tok/s on one core ({cpu['tokens_compared']} tokens, all equal to "
            f"the GPU's: {cpu['all_tokens_match_gpu']})")

    d, g, p = res.get("decode"), res.get("gemv"), res.get("prefill")
    line = {
        "metric": METRIC,
        "value": d["tok_s"] if d else None,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": d["ms_per_tok"] if d else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "cfg2: SmolLM2-360M-shaped Llama, Q8_0x4 weights N(0,0.02), KV pre-filled to 512, "
                               f"{args.steps} greedy decode tokens (one step = one token)",
                   "seq_len": CFG2["seq_len"], "start_pos": PREFILL_POS},
    }
    if g:
        traffic = measured_traffic()
        line["roofline"] = {"bound": "hbm", "achieved": round(g["achieved_gbs"], 1), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(g["achieved_gbs"] / HBM_PEAK_GBS, 4),
                            "traffic": round(traffic) if traffic else None,
                            "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT) if traffic else None,
                            "kernel": "k_gemv (Q8_0, M=1): the decode launches of a SmolLM2-1.7B-shaped model "
                                      "(fused QKV, O, fused gate+up, down x 24 layers + classifier), cold",
                            "avg_launch_us": round(g["avg_launch_us"], 3),
                            "read_ceiling": round(g["read_ceiling_gbs"], 1),
                            "frac_of_read_ceiling": round(g["achieved_gbs"] / g["read_ceiling_gbs"], 4),
                            "swept_read_ceiling": g["swept_read_ceiling"]["gbs"] if g["swept_read_ceiling"] else None,
                            "frac_of_swept_read_ceiling": (round(g["achieved_gbs"] / g["swept_read_ceiling"]["gbs"], 4)
                                                           if g["swept_read_ceiling"] else None),
                            "bytes_per_launch": round(g["bytes_per_launch"])}
        line["gemv"] = g
    if p:
        line["prefill"] = p
    if d:
        line["decode"] = d
    for key in ("cfg4", "cfg5"):
        if key in res:
            line[key] = res[key]
    if cpu:
        line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
