#!/usr/bin/env python3
"""Decode-step benchmark of the fused decode-on-codes KV attention on one MI355X.

A step is one decode-attention pass for every sequence of the batch over its
whole two-tier cache (K4 asym-NF4 + 2 % fp16 outliers, V3 PolarQuant, fp16 hot
window of 512).  The cache is pre-filled through the GPU encode path with
seeded synthetic fp16 keys/values of the measurement spec (lognormal
per-channel key scale, 2 % x10 channels, RoPE; N(0,1) values); queries are
fp16 N(0,1).  Inputs are resident in HBM before timing starts.  Several cache
replicas (>= 1 GB together) are used round-robin so the 256 MB Infinity Cache
cannot serve repeat steps.

Prints one JSON line.  `value` is microseconds per decode step (lower is
better), averaged over `--steps` back-to-back steps after a time-based
pre-roll (GPU clock ramp) and `--warmup` steps.  `roofline.achieved` is the
canonical compressed-KV bytes of one step divided by the average duration of
one decode-kernel launch (split-K over the coded groups and the hot window,
merged by its last workgroups: the whole step is this one launch), from the
timed region's HIP event pair on the launch stream around `--steps`
back-to-back steps.  `encode` holds the
prefill encode of the same workload and `cpu_baseline` the reference's CPU
decode path (oracle restatement) on this host's cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "turboquant-pro_amd"))

METRIC = "decode-attention µs/step + achieved HBM GB/s on codes, bs16×32K GQA-8"
HBM_PEAK_GBS = 8000.0

CONFIGS = {
    # the BASELINE metric's workload: Llama-3-8B GQA shape at batch 16 x 32K
    "headline": dict(B=16, Hkv=8, Hq=32, L=32768, vbits=3),
    "c1_8k": dict(B=16, Hkv=8, Hq=32, L=8192, vbits=3),
    "c2_128k": dict(B=1, Hkv=8, Hq=32, L=131072, vbits=3),
    "c0_mha4k": dict(B=1, Hkv=32, Hq=32, L=4096, vbits=4),
    "c4_70b": dict(B=32, Hkv=8, Hq=64, L=32768, vbits=3),
    # config 3: 64 sequences of seeded lengths U[1024, 32768], 16-token pages,
    # block table a seeded permutation of the physical pages
    "c3_paged_ragged": dict(B=64, Hkv=8, Hq=32, L=32768, vbits=3, ragged=True, page=16),
    # other key forms at the headline shape (not BASELINE configs): the
    # reference's default cache (bits=3: uniform 3-bit per-channel keys, no
    # outliers) and PolarQuant keys (per_channel_keys=False), both with V3
    "k3v3_default": dict(B=16, Hkv=8, Hq=32, L=32768, vbits=3, kbits=3, key_grid="uniform", ofrac=0.0),
    "k3v3_polar": dict(B=16, Hkv=8, Hq=32, L=32768, vbits=3, kbits=3, key_grid="polar", ofrac=0.0),
    # 4-bit keys without the side-list: asym-NF4 (the headline's keys minus
    # its outliers) and uniform (PerChannelKV's default grid)
    "k4v3_nf4_noout": dict(B=16, Hkv=8, Hq=32, L=32768, vbits=3, kbits=4, key_grid="nf4_asym", ofrac=0.0),
    "k4v3_uniform": dict(B=16, Hkv=8, Hq=32, L=32768, vbits=3, kbits=4, key_grid="uniform", ofrac=0.0),
    # pools the MFMA decode does not take, served by the VALU decode (split
    # kernel + merge kernel): head_dim 64, head_dim 256 (gemma-2-9b's 16 q /
    # 8 kv heads) and an fp32 cache (fp32 hot window and queries)
    "d64_8k": dict(B=16, Hkv=8, Hq=32, L=8192, vbits=3, D=64),
    "d256_8k": dict(B=16, Hkv=8, Hq=16, L=8192, vbits=3, D=256),
    "f32_8k": dict(B=16, Hkv=8, Hq=32, L=8192, vbits=3, dtype="float32"),
}


def mfma_config(cfg):
    """Whether the config's pool runs the MFMA decode (head_dim 128, fp16)."""
    return cfg.get("D", 128) == 128 and cfg.get("dtype", "float16") == "float16"


def config_lengths(cfg):
    """Sequence lengths of a config: all L, or the seeded ragged draw."""
    import numpy as np
    if cfg.get("ragged"):
        return [int(x) for x in np.random.default_rng(3).integers(1024, cfg["L"] + 1, size=cfg["B"])]
    return [cfg["L"]] * cfg["B"]


def n_groups(L, W=512):
    G = (W + 1) // 2
    return 0 if L <= W else (L - (W + 1)) // G + 1


def step_bytes(lens, Hkv, Hq, D=128, kbits=4, vbits=3, W=512, n_out=640, out_bytes=2, polar_keys=False,
               tok_bytes=2):
    """Canonical compressed bytes of one decode step (storage-of-record sizes):
    per (sequence, kv head) n_cold*(D*kb/8 + D*vb/8 + 4) + n_grp*(2*D*4 + n_out*6)
    + n_hot*2*D*tok_bytes, plus q in and output per query head.  PolarQuant
    keys carry a 4-byte norm per token instead of the per-group scale and mean;
    fp32 caches (tok_bytes 4) keep fp32 hot tokens and take fp32 queries."""
    G = (W + 1) // 2
    tot = 0
    for L in lens:
        ng = n_groups(L, W)
        n_cold, n_hot = ng * G, L - ng * G
        per_tok = D * kbits // 8 + D * vbits // 8 + 4 + (4 if polar_keys else 0)
        per_grp = (0 if polar_keys else 2 * D * 4) + n_out * 6
        tot += Hkv * (n_cold * per_tok + ng * per_grp + n_hot * 2 * D * tok_bytes
                      + (Hq // Hkv) * D * (tok_bytes + out_bytes))
    return tot


def key_form(cfg):
    """The key form of a config, in words."""
    grid = cfg.get("key_grid", "nf4_asym")
    kb = cfg.get("kbits", 4)
    if grid == "polar":
        return f"K{kb} PolarQuant keys"
    outl = " + 2% fp16 outliers" if cfg.get("ofrac", 0.02) > 0 else ""
    return f"K{kb} {'uniform per-channel' if grid == 'uniform' else 'asym-NF4'}{outl}"


def config_step_bytes(cfg):
    """step_bytes of a config: its key form, widths, head_dim, token width and
    outlier count (2 % of a 256-token group per channel: 5 x head_dim)."""
    D = cfg.get("D", 128)
    n_out = 5 * D if cfg.get("ofrac", 0.02) > 0 else 0
    return step_bytes(config_lengths(cfg), cfg["Hkv"], cfg["Hq"], D=D, kbits=cfg.get("kbits", 4),
                      vbits=cfg["vbits"], n_out=n_out, polar_keys=cfg.get("key_grid") == "polar",
                      tok_bytes=4 if cfg.get("dtype") == "float32" else 2)


def synth_chunk(torch, gen, scale, t0, n, B, Hkv, D=128, theta=10000.0, dtype=None):
    """fp16 (or ``dtype``) keys/values for positions [t0, t0+n): N(0,1) *
    per-channel scale, RoPE (rotate_half); values N(0,1)."""
    dev = scale.device
    k = torch.randn((B, Hkv, n, D), generator=gen, device=dev, dtype=torch.float32) * scale
    half = D // 2
    inv = theta ** (-2.0 * torch.arange(half, device=dev, dtype=torch.float64) / D)
    ang = torch.arange(t0, t0 + n, device=dev, dtype=torch.float64)[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], 1).float()
    sin = torch.cat([ang.sin(), ang.sin()], 1).float()
    rh = torch.cat([-k[..., half:], k[..., :half]], -1)
    dt = torch.float16 if dtype is None else dtype
    k = (k * cos + rh * sin).to(dt)
    v = torch.randn((B, Hkv, n, D), generator=gen, device=dev, dtype=torch.float32).to(dt)
    return k, v


def build_pool(torch, cfg, seed, chunk=4096):
    from turboquant_pro_amd import TQKVPool
    import numpy as np
    B, Hkv, Hq, L = cfg["B"], cfg["Hkv"], cfg["Hq"], cfg["L"]
    D, dtype = cfg.get("D", 128), cfg.get("dtype", "float16")
    lens = config_lengths(cfg)
    extra = {}
    if cfg.get("page"):
        P = cfg["page"]
        max_pages = n_groups(L) * 256 // P
        extra = dict(page_tokens=P, block_table=np.random.default_rng(4).permutation(B * max_pages).astype(np.int32))
    if "key_grid" in cfg:
        extra.update(key_grid=cfg["key_grid"], key_bits=cfg["kbits"], outlier_frac=cfg["ofrac"])
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, head_dim=D, max_batch=B, max_seq_len=L,
                    value_bits=cfg["vbits"], seed=seed, input_dtype=dtype, **extra)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    scale = torch.exp(torch.randn((B, Hkv, 1, D), generator=gen, device="cuda"))
    n_hot_ch = round(0.02 * D)
    for b in range(B):
        for h in range(Hkv):
            ch = torch.randperm(D, generator=gen, device="cuda")[:n_hot_ch]
            scale[b, h, 0, ch] *= 10.0
    t = 0
    while t < L:
        n = min(chunk, L - t)
        k, v = synth_chunk(torch, gen, scale, t, n, B, Hkv, D=D,
                           dtype=torch.float32 if dtype == "float32" else None)
        pool.append(k, v, n_new=[min(n, max(0, x - t)) for x in lens])
        t += n
    torch.cuda.synchronize()
    return pool


COPY_PROBE_BYTES = 256 << 20


def measured_traffic(config):
    """HBM bytes per launch of the split kernel on this workload, read from the
    committed counter profile profiles/tqk_decode_split_mfma_<config>_traffic.md
    (FETCH_SIZE / WRITE_SIZE passes, each scaled by its reading on a plain copy
    of known size).  It is not counted in this run: the profile names the build
    it was measured on.  Returns (bytes or None, source text)."""
    import re
    name = f"tqk_decode_split_mfma_{config}_traffic.md"
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None, "not measured for this config"
    m = re.search(r"traffic_bytes_per_launch\s*=\s*(\d+)", text)
    b = re.search(r"build_commit\s*=\s*(\w+)", text)
    src = f"committed counter profile profiles/{name}" + (f" (build {b.group(1)})" if b else "") + \
        ", not counted in this run"
    return (int(m.group(1)) if m else None), src


_CPU_STATE = {}


def _cpu_pair_attend(i):
    """One (sequence, kv head) pair's dequantize-then-attend (pool worker)."""
    sc, q = _CPU_STATE["cache"], _CPU_STATE["q"]
    out = sc.attend(q)
    return float(out[0, 0])


def cpu_workers():
    """Worker processes for the CPU baseline: the host cores this process may
    run on, at most 16 (one GPU's share of a box)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(cfg, steps=3):
    """The reference CPU decode path as the oracle restates it (NumPy
    dequantize-then-attend, turboquant_pro/core.py:1040-1117 +
    per_channel_kv.py:497-539 + core.py:619-654), timed on this host for whole
    decode steps: every (sequence, kv head) pair of the batch attends over its
    full-context cache, the pairs spread over a pool of single-threaded worker
    processes (NumPy/BLAS one thread each).  All pairs use one synthetic pair
    cache of the workload's context (the cost of a pair does not depend on its
    data).  Median of ``steps`` whole steps.  Runs before the GPU is touched:
    the workers are forked from a process that has not initialised HIP."""
    import multiprocessing as mp
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import tq_oracle as O
    L, g = cfg["L"], cfg["Hq"] // cfg["Hkv"]
    t0 = time.perf_counter()
    k, v, q = O.synthetic_kv(1, 1, 1, g, L)
    pi, pi_t = O.rotation(0, 128)
    sc = O.SequenceCache(hot_window=512, value_bits=cfg["vbits"], outlier_frac=0.02).build(
        k[0], v[0], pi, pi_t)
    build_s = time.perf_counter() - t0
    _CPU_STATE["cache"], _CPU_STATE["q"] = sc, q[0]
    pairs = cfg["B"] * cfg["Hkv"]
    nw = cpu_workers()
    times = []
    with mp.get_context("fork").Pool(nw) as pool:
        pool.map(_cpu_pair_attend, range(nw))  # workers up and warm
        for _ in range(steps):
            t1 = time.perf_counter()
            res = pool.map(_cpu_pair_attend, range(pairs), chunksize=1)
            times.append(time.perf_counter() - t1)
    assert np.isfinite(res).all()
    step_s = float(np.median(times))
    return {"value": round(step_s * 1e6, 1), "unit": "us/step", "cores": nw, "kind": "port",
            "sample": f"median of {steps} whole decode steps: {pairs} (sequence, kv head) pairs x "
                      f"L={L} with {g} q-heads each, over {nw} worker processes x 1 NumPy/BLAS "
                      f"thread (steps {', '.join(f'{t * 1e3:.0f}' for t in times)} ms; pair cache "
                      f"built once in {build_s:.1f} s, encode excluded); cpu={_cpu_model()}, "
                      f"os.cpu_count()={os.cpu_count()}"}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


VALU_OPS_PEAK = 256 * 4 * 16 * 2.4e9  # separately rounded fp32 ops/s: 256 CUs x 4 SIMD x 16 lanes x 2.4 GHz


def encode_bench(torch, cfg, fills, chunk=4096):
    """Prefill encode: the config's batch appended in ``chunk``-token chunks up
    to its context (group flushes through the encode kernel, hot-ring copies),
    ``fills`` times after one untimed fill; median fill.  Bytes: fp16 K+V in
    (512 B per token-head) + the coded groups out in the reference's container
    sizes (116 B per cold token-head at K4/V3 plus 4864 B of stats and
    side-list per group-head).  The encode is bound by
    the value rotation's 2 * 128^2 separately rounded fp32 operations per
    token-head (no FMA, no packed math: the bit-exactness contract), reported
    against the chip's unpacked VALU issue rate."""
    from turboquant_pro_amd import TQKVPool
    B, Hkv, Hq, L, vb = cfg["B"], cfg["Hkv"], cfg["Hq"], cfg["L"], cfg["vbits"]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    scale = torch.exp(torch.randn((B, Hkv, 1, 128), generator=gen, device="cuda"))
    chunks = [synth_chunk(torch, gen, scale, t, min(chunk, L - t), B, Hkv) for t in range(0, L, chunk)]
    kf = (dict(key_grid=cfg["key_grid"], key_bits=cfg["kbits"], outlier_frac=cfg["ofrac"])
          if "key_grid" in cfg else {})
    pool = TQKVPool(n_kv_heads=Hkv, n_q_heads=Hq, max_batch=B, max_seq_len=L, value_bits=vb, seed=0, **kf)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for it in range(fills + 1):
        pool.reset()
        torch.cuda.synchronize()
        e0.record()
        for k, v in chunks:
            pool.append(k, v)
        e1.record()
        torch.cuda.synchronize()
        if it:
            times.append(e0.elapsed_time(e1))
    ms = sorted(times)[len(times) // 2]
    n_cold = n_groups(L) * ((512 + 1) // 2)
    kb = cfg.get("kbits", 4)
    polar = cfg.get("key_grid") == "polar"
    n_out = 640 if cfg.get("ofrac", 0.02) > 0 else 0
    per_token = 128 * kb // 8 + 128 * vb // 8 + 4 + (4 if polar else 0)
    per_group = 0 if polar else 2 * 128 * 4 + n_out * 6
    nbytes = B * Hkv * (L * 2 * 128 * 2 + n_cold * per_token) + B * Hkv * n_groups(L) * per_group
    # PolarQuant keys go through the same rotation as the values
    rot_ops = B * Hkv * n_cold * 2 * 128 * 128 * (2 if polar else 1)
    return {"metric": "prefill encode GB/s (fp16 K+V in + coded groups out)",
            "value": round(nbytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s",
            "ms_per_fill": round(ms, 3), "tokens_per_s": round(B * L / (ms * 1e-3)),
            "fills": len(times), "bytes": nbytes,
            "rotation_ops_per_s": round(rot_ops / (ms * 1e-3) / 1e12, 2),
            "valu_frac": round(rot_ops / (ms * 1e-3) / VALU_OPS_PEAK, 3),
            "config": {"name": cfg.get("name", ""), "batch": B, "context": L, "n_kv_heads": Hkv,
                       "chunk": chunk, "value_bits": vb, "keys": key_form(cfg)}}


def preroll(fn, min_ms):
    """Untimed decode launches until ``min_ms`` of wall time have passed (and
    the GPU has drained them): the GPU clocks ramp over the first tens of ms of
    sustained work, so the timed steps start at steady state whatever
    ``--warmup`` is.  Returns (launches, elapsed ms)."""
    import torch
    n = 0
    t0 = time.perf_counter()
    while True:
        for _ in range(20):
            fn(n)
            n += 1
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3
        if ms >= min_ms:
            return n, ms


def block_bench(torch, steps, S=32768, H=8, D=128):
    """The block store's whole-request key save: ``tqk_encode_key_block`` (the
    ``per_channel`` plugin's compress, turboquant_pro/per_channel_kv.py:285-401)
    on one (1, H, S, D) fp16 block, asym-NF4 + 2 % outliers, each (b, h) one
    group.  Bytes: fp16 keys in + 4-bit codes, per-channel scale and mean and
    the side-list (6 B an entry) out.  Median of ``steps`` timed calls after
    one untimed call."""
    import ctypes
    import statistics
    from turboquant_pro_amd import _native as N
    from turboquant_pro_amd.codebooks import outliers_per_channel
    from turboquant_pro_amd.plugins import _block_desc
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    x = (torch.randn((1, H, S, D), generator=gen, device="cuda") *
         torch.exp(0.5 * torch.randn((1, H, 1, D), generator=gen, device="cuda"))).half()
    k = outliers_per_channel(S, 0.02)
    cap = min(S * D, 4 * k * D)
    kp = torch.empty(H * S * D // 2, dtype=torch.uint8, device="cuda")
    scale = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
    zero = torch.empty_like(scale)
    count = torch.zeros(H, dtype=torch.int32, device="cuda")
    pos = torch.empty((H, cap), dtype=torch.int32, device="cuda")
    val = torch.empty((H, cap), dtype=torch.float16, device="cuda")
    d = _block_desc(x.shape, 4, 0, 0, k, cap, 0, None)
    st = torch.cuda.current_stream()

    def call():
        N.check(N.lib().tqk_encode_key_block(
            ctypes.byref(d), x.data_ptr(), None, kp.data_ptr(), scale.data_ptr(), zero.data_ptr(),
            pos.data_ptr(), val.data_ptr(), count.data_ptr(), ctypes.c_void_p(st.cuda_stream)),
            "tqk_encode_key_block")

    call()
    torch.cuda.synchronize()
    n_out = int(count.sum().item())
    times = []
    for _ in range(max(steps, 1)):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        call()
        e1.record(st)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    ms = statistics.median(times)
    nbytes = H * S * D * 2 + H * S * D // 2 + H * D * 8 + n_out * 6
    return {"metric": "block key encode ms + GB/s (fp16 keys in, codes and side-list out)",
            "value": round(ms, 3), "unit": "ms", "higher_is_better": False,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes, "calls": len(times),
            "workgroups": H, "outliers": n_out,
            "config": {"workload": f"tqk_encode_key_block, one (1, {H}, {S}, {D}) fp16 block, "
                                   "asym-NF4 + 2% outliers"},
            "data": "synthetic (seeded N(0,1) x lognormal per-channel scale, fp16)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--preroll-ms", type=float, default=300.0,
                    help="untimed, time-based run of decode launches before the warm-up "
                         "(GPU clock ramp), reported as preroll_ms")
    ap.add_argument("--config", default="headline", choices=sorted(CONFIGS))
    ap.add_argument("--replicas", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-encode", action="store_true",
                    help="skip the prefill-encode sub-record of the decode line")
    ap.add_argument("--encode", action="store_true",
                    help="measure the prefill encode instead (quantize-on-append of 4096-token chunks "
                         "of the chosen config; prints its own JSON line, not the decode metric)")
    ap.add_argument("--block", action="store_true",
                    help="measure the plugins' stateless key-block encode on one (1, 8, 32768, 128) "
                         "block instead (prints its own JSON line)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="after timing, copy a 256 MiB buffer 3 times (calibration kernel for "
                         "the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the decode shards by "
                          "(sequence, kv head) with no communication, but multi-GPU runs are "
                          "out of scope here", "n_gpus": args.gpus}))
        sys.exit(2)

    if args.block:
        import torch
        print(json.dumps(block_bench(torch, min(args.steps, 10))), flush=True)
        return
    cfg = CONFIGS[args.config]
    if args.encode and not mfma_config(cfg):
        print(json.dumps({"error": "the encode bench covers head_dim 128 fp16 configs only"}))
        sys.exit(2)
    cpu = None
    if not args.encode and not args.no_cpu_baseline and "key_grid" not in cfg and mfma_config(cfg):
        # single-threaded BLAS in each worker process; set before NumPy loads
        for var in ("OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS"):
            os.environ[var] = "1"
        t0 = time.time()
        cpu = cpu_baseline(cfg)
        print(f"[bench] cpu baseline done in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    import torch

    if args.encode:
        print(json.dumps(encode_bench(torch, dict(cfg, name=args.config), args.steps)), flush=True)
        return
    B, Hkv, Hq, L = cfg["B"], cfg["Hkv"], cfg["Hq"], cfg["L"]
    print(f"[bench] config={args.config} {cfg} replicas={args.replicas}", file=sys.stderr, flush=True)
    t0 = time.time()
    pools = [build_pool(torch, cfg, seed=1000 + r) for r in range(args.replicas)]
    print(f"[bench] prefill done in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    D = cfg.get("D", 128)
    f32 = cfg.get("dtype") == "float32"
    q = torch.randn((B, Hq, D), generator=gen, device="cuda")
    q = q if f32 else q.half()
    outs = [torch.empty((B, Hq, D), dtype=torch.float32, device="cuda") for _ in pools]

    def step(i):
        pools[i % len(pools)].decode(q, out=outs[i % len(pools)])

    n_pre, pre_ms = preroll(step, args.preroll_ms)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps

    # the kernel's average launch duration: each step of an MFMA config is
    # exactly one tqk_decode launch (the in-kernel merge writes the output),
    # so the event pair around the `steps` back-to-back launches of the timed
    # region, divided by `steps`, is the average launch duration; the kernel
    # trace of the same command (rocprofv3 --kernel-trace) cross-checks it.
    # A VALU config's step is two launches (split kernel, merge kernel).
    kernel_ms = ms_per_step
    nbytes = config_step_bytes(cfg)
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    step_gbs = nbytes / (ms_per_step * 1e-3) / 1e9

    if args.copy_probe:
        src = torch.empty(COPY_PROBE_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": COPY_PROBE_BYTES, "copies": 3}), file=sys.stderr, flush=True)

    traffic, traffic_src = measured_traffic(args.config)

    enc = None
    if not args.no_encode and mfma_config(cfg):
        del pools
        torch.cuda.empty_cache()
        enc = encode_bench(torch, dict(cfg, name=args.config), 5)

    line = {
        "metric": METRIC,
        "value": round(ms_per_step * 1e3, 2),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "preroll_ms": round(pre_ms, 1),
        "preroll_launches": n_pre,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": f"synthetic (seeded lognormal-scaled RoPE {'fp32' if f32 else 'fp16'} keys with 2% x10 "
                "channels, N(0,1) values and queries), cache filled through the GPU encode path",
        "config": {"workload": f"decode step, batch {B} x context "
                               + (f"U[1024, {L}] (seeded, mean {sum(config_lengths(cfg)) // B}), "
                                  f"{cfg['page']}-token pages, permuted block table"
                                  if cfg.get("ragged") else f"{L}")
                               + f", {Hq} q-heads / {Hkv} kv-heads, "
                               f"head_dim {D}, {key_form(cfg)}, V{cfg['vbits']} "
                               f"PolarQuant, {'fp32' if f32 else 'fp16'} hot window 512",
                   "name": args.config, "batch": B, "context": L, "n_q_heads": Hq,
                   "n_kv_heads": Hkv, "replicas": args.replicas},
        "step_bytes": nbytes,
        "step_gbs": round(step_gbs, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": "tqk_decode_split_mfma" if mfma_config(cfg)
                               else "tqk_decode_split_valu + tqk_merge",
                     "kernel_us": round(kernel_ms * 1e3, 2),
                     "kernel_us_method": f"the timed region: one HIP event pair on the launch "
                                         f"stream around {args.steps} back-to-back decode steps "
                                         + ("of one tqk_decode launch each" if mfma_config(cfg)
                                            else "of two launches each (split, merge)")
                                         + f", divided by {args.steps}"},
        "encode": enc,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
