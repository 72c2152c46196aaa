#!/usr/bin/env python3
"""Benchmark of the MI355X paged decode attention path.

Metric: paged decode attn -- us/step and achieved HBM GB/s (% of the 8 TB/s
peak) at B=32, one MI355X.

Workload (default `batch32_mixed`): B=32 sequences, Qwen2.5-0.5B heads
(14 q / 2 kv, head_dim 64), fp16, contexts U{128..4096} (seeded), page size 16,
16384-page pool handed out by a seeded shuffle, 24 layers.  A step is one
layer's decode step for the whole batch (luc_decode_step, one launch): RoPE(q,
k) + paged append of one new token per sequence, split-K paged attention whose
last split per sequence merges the partials (log-sum-exp).  Successive steps
walk the 24 layers (all of them when K >= 24) so the working set (~830 MB at 24
layers) does not fit the 256 MB Infinity Cache.  Inputs are resident in HBM
before timing; the K steps are captured in one HIP graph, replayed three
times untimed and then three times timed, each timed replay bracketed by
torch.cuda.synchronize(); ms_per_step is the median replay over K.

Also reported:
  roofline      the paged decode operation (luc_paged_decode: the split-K
                decode kernel, merge included): algorithmic bytes per
                launch (K+V over every context token, q, output, block table)
                over its average duration, measured with HIP events around a
                graph of back-to-back launches on the launch stream;
                `traffic` is the HBM bytes per launch read from the committed
                rocprofv3 PMC summary, if that summary measured the code
                object loaded now (its SHA-256 matches), else null;
  cpu_baseline  the oracle (C restatement of the reference's attention, OpenMP)
                on one full layer step of the same workload on the host, on the
                process's CPU share (the cores it may run on, at most the
                OMP_NUM_THREADS the box sets for one GPU) and (single_core) on
                one, with nproc and the affinity count stated; `single_512`
                is the same for the single-sequence workload (B=1, ctx 512,
                14q/2kv, fp16), the one the reference's own path serves;
  long_context  the paged decode operation (luc_paged_decode) on
                batch64_long (B=64, 28q/4kv, d=128, bf16, ctx U{1024..16384};
                the automatic split and the configuration's 512-token split)
                and batch8_32k (B=8, 12q/2kv, d=128, bf16, ctx 32768), 4
                layers rotated, per launch: us, algorithmic GB/s, fraction
                of 8 TB/s, and the two memory floors below for the same
                bytes (the gather with 4-tile workgroups, not the long
                splits the decode kernel uses there);
  floors        (in roofline) luc_gather_floor: the same K/V page slabs as
                the decode kernel reads, with its work split and no
                arithmetic, and luc_stream_read: the same bytes read
                contiguously -- the memory floors under the kernel;
  prefill       luc_paged_prefill on prefill_4x2048 (4 prompts x 2048 rows from
                an empty cache, 14q/2kv, d=64, bf16): RoPE + cache append
                kernel, then the causal attention kernel on bf16 MFMA; time per
                call (HIP events over a graph of back-to-back calls) and the
                attention's algorithmic FLOP rate against the 2.5 PFLOP/s dense
                bf16 peak; mfma_busy_frac is the share of SIMD cycles with the
                matrix cores busy, from the committed rocprofv3 PMC summary
                (null unless it measured the code object loaded now);
  code_objects  the first 16 hex digits of the SHA-256 of each code object
                the measured kernels come from;
  sampling      luc_sort_and_sample on one logits row (vocab 151936, top_k
                1024): time per call;
  model         the Qwen2 model loop (random-init Qwen2.5-0.5B, bf16, B=1):
                a 128-token prompt, then greedy decode steps replayed from one
                HIP graph (Qwen2Model.capture_decode: 24 layers of RMSNorm,
                qkv GEMM, luc_decode_step, o_proj, RMSNorm, gate|up GEMM,
                silu*up, down_proj; final norm, lm_head, argmax), time per
                token and the bytes each token reads (every weight once plus
                the K/V of its context) against 8 TB/s; also the eager,
                host-driven loop's time per token.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_batch32_mixed_traffic.json")
MFMA_FILE = os.path.join(ROOT, "profiles", "prefill_4x2048_mfma.json")
CODE_DIR = os.path.join(ROOT, "lucciola-rs_amd", "lib")


def code_object_sha256(name):
    """SHA-256 of the machine code of the gfx950 code object lib/<name>.hsaco
    that the library loads: its .text (the kernels' instructions) and .rodata
    (their kernel descriptors: register counts, LDS size) sections, in that
    order (None if it is not built).  The rest of the file (symbol tables)
    names hipcc's temporary files and so differs from build to build of the
    same source."""
    import hashlib
    import struct
    path = os.path.join(CODE_DIR, name + ".hsaco")
    if not os.path.exists(path):
        return None
    with open(path, "rb") as f:
        elf = f.read()
    if elf[:4] != b"\x7fELF" or elf[4] != 2 or elf[5] != 1:
        return None  # not a little-endian ELF64 file
    shoff, = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", elf, 0x3A)
    secs = [struct.unpack_from("<IIQQQQ", elf, shoff + i * shentsize) for i in range(shnum)]
    strtab_off = secs[shstrndx][4]

    def name_of(sec):
        start = strtab_off + sec[0]
        return elf[start:elf.index(b"\0", start)].decode()

    by_name = {name_of(sec): sec for sec in secs}
    h = hashlib.sha256()
    for sec_name in (".text", ".rodata"):
        sec = by_name.get(sec_name)
        if sec is None:
            return None
        h.update(elf[sec[4]:sec[4] + sec[5]])
    return h.hexdigest()


def profile_value(path, key):
    """`key` of a committed rocprofv3 PMC summary, or None when the summary is
    missing or was measured on another build of its code object: the summary
    names the code object and the SHA-256 it measured ("code_object",
    "code_object_sha256"), and a figure is used only if that hash equals the
    hash of the code object loaded now."""
    if not os.path.exists(path):
        return None
    with open(path) as f:
        prof = json.load(f)
    name, sha = prof.get("code_object"), prof.get("code_object_sha256")
    if not name or not sha or code_object_sha256(name) != sha:
        return None
    return prof.get(key)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=480)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--workload", default="batch32_mixed")
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--eager", action="store_true", help="launch eagerly instead of a HIP graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-long-context", action="store_true",
                    help="skip the batch64_long / batch8_32k decode measurements")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the prefill and sampling measurements")
    ap.add_argument("--no-model", action="store_true",
                    help="skip the Qwen2 model loop measurement")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a 1 GiB device copy (reference for PMC byte counters)")
    return ap.parse_args()


def cpu_share():
    """(threads, nproc, affinity): the cores this process may run on
    (sched_getaffinity), capped by OMP_NUM_THREADS where the box sets it (its
    CPU share per GPU), and the machine's nproc."""
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(affinity, omp) if omp > 0 else affinity
    return max(threads, 1), os.cpu_count(), affinity


def cpu_baseline(cfg, seed, budget_s=10.0, threads=None):
    """Time the oracle's decode step (one layer, the whole batch) on the host
    with `threads` OpenMP threads (default: the process's CPU share)."""
    import oracle
    from lucciola_rs_amd import workloads as wl
    from lucciola_rs_amd.engine import sm_scale

    if threads is None:
        threads = cpu_share()[0]
    h = wl.host_decode_inputs(cfg, seed, num_layers=1, poison=False)
    orc = oracle.get()
    cos, sin = orc.rope_table(cfg.ctx_hi + 1, cfg.head_dim, cfg.rope_theta)

    def run():
        qkv, kp, vp = h.qkv.copy(), h.k_pool.copy(), h.v_pool.copy()
        t0 = time.perf_counter()
        orc.decode_step(qkv, None, None, None, cos, sin, kp, vp, h.tables, h.positions, 0, cfg.hq,
                        cfg.hkv, cfg.head_dim, sm_scale(cfg.head_dim), 16, 1, cfg.dtype,
                        threads)
        return time.perf_counter() - t0

    run()  # warm-up
    times, start = [], time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - start < budget_s and len(times) < 20):
        times.append(run())
    t = statistics.median(times)
    return dict(t=t, threads=threads, reps=len(times), ctx=h.ctx)


def prefill_bench(lib, torch, reps=50):
    """Microseconds per luc_paged_prefill call on prefill_4x2048, replayed from
    a HIP graph, and the attention's algorithmic FLOPs."""
    import numpy as np
    from lucciola_rs_amd import workloads as wl
    from lucciola_rs_amd.engine import RopeCache, sm_scale

    cfg = wl.PREFILL_CONFIGS["prefill_4x2048"]
    h = wl.host_prefill_inputs(cfg, seed=1, poison=False)
    dev = torch.device("cuda:0")
    to = lambda x: wl.bits_to_tensor(np.ascontiguousarray(x), cfg.dtype).to(dev)
    qkv, kp, vp = to(h.qkv), to(h.k_pool), to(h.v_pool)
    tables = torch.from_numpy(h.tables).to(dev)
    cu = torch.from_numpy(h.cu_seqlens).to(dev)
    sp = torch.from_numpy(h.start_pos).to(dev)
    rope = RopeCache(4096, cfg.head_dim, 1e6, lib=lib, device=dev)
    total = int(h.cu_seqlens[-1])
    out = torch.empty((total, cfg.hq * cfg.head_dim), dtype=cfg.torch_dtype, device=dev)

    def call():
        # q/k are roped in place on every call: the same work each time
        lib.paged_prefill(qkv, None, None, None, rope.cos, rope.sin, kp, vp, tables, cu, sp, total,
                          h.max_ctx, 0, 1, cfg.hq, cfg.hkv, cfg.head_dim, sm_scale(cfg.head_dim), out)

    for _ in range(5):
        call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            call()
    g.replay()
    torch.cuda.synchronize()
    runs = []
    for _ in range(5):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        runs.append(e0.elapsed_time(e1) * 1e3 / reps)
    us = statistics.median(runs)
    flops = wl.prefill_flops(cfg, np.diff(h.cu_seqlens), h.start_pos)
    tflops = flops / (us * 1e-6) / 1e12
    return {"workload": cfg.name, "batch": cfg.batch, "rows": cfg.rows, "q_heads": cfg.hq,
            "kv_heads": cfg.hkv, "head_dim": cfg.head_dim, "dtype": cfg.dtype,
            "call": "luc_paged_prefill (RoPE + append kernel, causal attention kernel)",
            "us_per_call": round(us, 2), "attention_flops": int(flops),
            "achieved_tflops": round(tflops, 1), "peak_tflops": PEAK_BF16_TFLOPS,
            "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "mfma_busy_frac": mfma_busy()}


def mfma_busy():
    """Fraction of SIMD cycles with the matrix cores busy during the prefill
    attention kernel, from the committed rocprofv3 PMC summary (None unless it
    measured the code object loaded now)."""
    return profile_value(MFMA_FILE, "mfma_busy_frac")


def sampling_bench(lib, torch, reps=100):
    """Microseconds per luc_sort_and_sample call (top-k filter + sort/sample
    kernels) on one Qwen2.5 logits row (vocab 151936, bf16, seeded N(0,1)*4),
    top_k 1024, top_p 0.9, replayed from a HIP graph."""
    import numpy as np
    from lucciola_rs_amd import workloads as wl

    vocab, top_k = 151936, 1024
    rng = np.random.default_rng(3)
    logits = wl.bits_to_tensor(wl.to_bits(rng.standard_normal(vocab) * 4, "bf16"), "bf16").cuda()
    buf = torch.zeros(2 * top_k, dtype=torch.int32, device="cuda")
    idx = torch.zeros(1, dtype=torch.int32, device="cuda")

    def call():
        lib.sort_and_sample(logits, 0.9, top_k, 0.37, buf, idx)

    for _ in range(3):
        call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            call()
    g.replay()
    torch.cuda.synchronize()
    runs = []
    for _ in range(5):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        runs.append(e0.elapsed_time(e1) * 1e3 / reps)
    return {"call": "luc_sort_and_sample (top-k filter + bitonic sort / top-p draw)",
            "vocab": vocab, "top_k": top_k, "top_p": 0.9,
            "us_per_call": round(statistics.median(runs), 2)}


def model_bench(lib, torch, prompt_len=128, steps=128, eager_steps=8):
    """Milliseconds per greedy token of the Qwen2.5-0.5B model loop (random
    init, B=1): prompt, eager steps (which also set up the GEMM handles), then
    a graph of one decode step replayed `steps` times, timed with HIP events."""
    import numpy as np
    from lucciola_rs_amd.model import QWEN25_05B, Qwen2Model, random_weights

    cfg = QWEN25_05B
    max_ctx = 512
    m = Qwen2Model(cfg, random_weights(cfg, seed=2025), max_positions=max_ctx, lib=lib)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, cfg.vocab_size, prompt_len).tolist()
    m.forward(prompt, 0)
    tok, pos = m.sample_greedy(), prompt_len
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(eager_steps):
        m.forward([tok], pos)
        tok, pos = m.sample_greedy(), pos + 1
    eager_ms = (time.perf_counter() - t0) * 1e3 / eager_steps
    graph = m.capture_decode(max_ctx)
    m.pos.fill_(pos)  # m.idx holds the last token
    for _ in range(4):
        graph.replay()
    torch.cuda.synchronize()
    ctx0 = pos + 4
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # what a token reads: the one-row products' weights ([out, in], "*_w"),
    # norms and biases (the transposed copies "*_t" serve prompts only)
    weights = sum(t.numel() * t.element_size() for t in
                  [m.lm_head_w, m.final_norm] +
                  [x for L in m.layers for k, x in L.items() if not k.endswith("_t")])
    mean_ctx = ctx0 + (steps + 1) / 2
    kv = int(mean_ctx) * cfg.num_hidden_layers * 2 * cfg.num_key_value_heads * cfg.head_dim * 2
    per_token = weights + kv
    # the largest one-row product alone: the final norm + lm_head GEMV
    # (luc_rmsnorm_gemv, 151936 x 896), 20 calls per graph, median of
    # replays; alternate calls read a copy of the weights, so that no call
    # finds the previous one's 272 MB in the 256 MB last-level cache
    logits = torch.empty(1, m.lm_head_w.shape[0], dtype=torch.bfloat16, device=m.device)
    heads = [m.lm_head_w, m.lm_head_w.clone()]
    lm_us = graph_us(torch, lambda i: lib.rmsnorm_gemv(logits, m.hidden, m.final_norm,
                                                       cfg.rms_norm_eps, heads[i % 2]), 20)
    del heads
    lm_bytes = (m.lm_head_w.numel() + logits.numel() + 2 * m.hidden.numel()) * 2
    del graph, m
    torch.cuda.empty_cache()
    return {"workload": "qwen2.5-0.5b greedy decode (random init, bf16, B=1, 24 layers)",
            "prompt": prompt_len, "steps": steps, "mean_ctx": round(mean_ctx, 1),
            "launch": "hip graph of one decode step (Qwen2Model.capture_decode)",
            "ms_per_token": round(ms, 4), "tokens_per_s": round(1e3 / ms, 1),
            "bytes_per_token": int(per_token), "achieved_gbs": round(per_token / (ms * 1e-3) / 1e9, 1),
            "frac": round(per_token / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "eager_ms_per_token": round(eager_ms, 3),
            "lm_head_gemv": {"kernel": "luc_rmsnorm_gemv_bf16_r8c2", "us_per_call": round(lm_us, 2),
                             "bytes": int(lm_bytes), "achieved_gbs": round(lm_bytes / (lm_us * 1e-6) / 1e9, 1),
                             "frac": round(lm_bytes / (lm_us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}}


def graph_us(torch, fn, n, reps=5, warm=3):
    """Median microseconds per call of fn(i), i < n, replayed from a HIP graph
    after `warm` untimed replays (the first replays of a graph over freshly
    allocated pools run several microseconds per call slower)."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    for _ in range(warm):
        g.replay()
    torch.cuda.synchronize()
    runs = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        runs.append(e0.elapsed_time(e1) * 1e3 / n)
    return statistics.median(runs)


def long_context_bench(lib, torch, name, seed, layers=4, launches=40, split_tokens=0):
    """luc_paged_decode on a long-context workload: us per launch (graph of
    back-to-back launches over `layers` rotated layers), algorithmic GB/s
    and fraction of the 8 TB/s peak.  split_tokens 0 is the library's
    automatic split; 512 is the split the batch64_long configuration names
    (8..32 splits per sequence of its longer contexts)."""
    import numpy as np
    from lucciola_rs_amd import workloads as wl
    from lucciola_rs_amd.engine import sm_scale

    cfg = wl.CONFIGS[name]
    dev = torch.device("cuda:0")
    inp = wl.device_decode_inputs(cfg, seed, layers, device=dev)
    ctx = inp["ctx"]
    max_ctx = int(ctx.max())
    out = torch.empty((cfg.batch, cfg.hq * cfg.head_dim), dtype=cfg.torch_dtype, device=dev)
    ws = lib.workspace(cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim, max_ctx, split_tokens)

    def call(i):
        lib.paged_decode(out, inp["qkv"], inp["k_pool"], inp["v_pool"], inp["tables"],
                         inp["positions"], cfg.batch, max_ctx, i % layers, layers, cfg.hq, cfg.hkv,
                         cfg.head_dim, sm_scale(cfg.head_dim), split_tokens, ws,
                         out_row_stride=out.shape[-1], q_row_stride=cfg.row)

    for i in range(layers):
        call(i)
    torch.cuda.synchronize()
    us = graph_us(torch, call, launches)
    nbytes = wl.decode_bytes(cfg, ctx) - cfg.batch * cfg.hkv * cfg.head_dim * 2 * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    res = {"workload": name, "batch": cfg.batch, "q_heads": cfg.hq, "kv_heads": cfg.hkv,
           "head_dim": cfg.head_dim, "dtype": cfg.dtype, "mean_ctx": float(np.mean(ctx)),
           "layers_rotated": layers, "split_tokens": split_tokens or "auto",
           "us_per_launch": round(us, 2),
           "algorithmic_bytes_per_launch": int(nbytes), "achieved_gbs": round(gbs, 1),
           "frac": round(gbs / PEAK_HBM_GBS, 4)}
    res.update(floors(lib, torch, cfg, inp, max_ctx, layers, nbytes, launches=launches))
    del inp
    torch.cuda.empty_cache()
    return res


def floors(lib, torch, cfg, inp, max_ctx, layers, nbytes, launches=240):
    """Memory floors under the decode kernel at this workload: the page-slab
    gather with the decode kernel's split and no arithmetic, and the same
    number of bytes read contiguously (from the K pool, offsets rotated so
    successive reads do not hit the same 256 MB)."""
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")

    def gather(i):
        lib.gather_floor(inp["k_pool"], inp["v_pool"], inp["tables"], inp["positions"], cfg.batch,
                         max_ctx, i % layers, layers, cfg.hkv, cfg.head_dim, sink)

    flat = inp["k_pool"].view(-1)
    n = (nbytes // 2 // 8) * 8  # elements, a multiple of 16 bytes
    span = flat.numel() - n

    def contiguous(i):
        off = ((i % layers) * (span // max(layers, 1))) // 8 * 8
        lib.stream_read(flat[off:off + n], sink)

    for i in range(layers):
        gather(i)
        contiguous(i)
    torch.cuda.synchronize()
    g = graph_us(torch, gather, launches)
    c = graph_us(torch, contiguous, launches)
    return {"gather_floor_us": round(g, 3), "gather_floor_gbs": round(nbytes / (g * 1e-6) / 1e9, 1),
            "contiguous_read_us": round(c, 3),
            "contiguous_read_gbs": round(nbytes / (c * 1e-6) / 1e9, 1)}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the paged decode path is a single-GPU kernel and no multi-GPU run is provided.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import __graft_entry__
    pkg = __graft_entry__.load_package()
    from lucciola_rs_amd import workloads as wl
    from lucciola_rs_amd.engine import RopeCache, decode_step, sm_scale

    cfg = wl.CONFIGS[args.workload]
    L = args.layers
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = pkg.library.default(0)
    inp = wl.device_decode_inputs(cfg, args.seed, L, device=dev)
    ctx = inp["ctx"]
    max_ctx = int(ctx.max())
    rope = RopeCache(max(max_ctx, 4096), cfg.head_dim, cfg.rope_theta, lib=lib, device=dev)
    out = torch.empty((cfg.batch, cfg.hq * cfg.head_dim), dtype=cfg.torch_dtype, device=dev)
    ws = lib.workspace(cfg.batch, cfg.hq, cfg.hkv, cfg.head_dim, max_ctx, args.split_tokens)
    qkv, kp, vp = inp["qkv"], inp["k_pool"], inp["v_pool"]
    tables, pos = inp["tables"], inp["positions"]

    def step(i):
        decode_step(qkv, None, None, None, rope, kp, vp, tables, pos, max_ctx, i % L, L, cfg.hq,
                    cfg.hkv, cfg.head_dim, out, ws, args.split_tokens, lib=lib)

    def decode_only(i):
        lib.paged_decode(out, qkv, kp, vp, tables, pos, cfg.batch, max_ctx, i % L, L, cfg.hq,
                         cfg.hkv, cfg.head_dim, sm_scale(cfg.head_dim), args.split_tokens, ws,
                         out_row_stride=out.shape[-1], q_row_stride=cfg.row)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    def timed(fn, n, reps=3):
        """Milliseconds for n calls of fn, launched eagerly or replayed from a
        graph: the median of `reps` timed runs of the n calls, each bracketed
        by synchronizations (graphs: after three untimed replays, the first of
        which uploads the graph)."""
        runs = []
        g = None
        if not args.eager:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(n):
                    fn(i)
            for _ in range(3):
                g.replay()
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            if g is None:
                for i in range(n):
                    fn(i)
            else:
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            runs.append(e0.elapsed_time(e1))
        return statistics.median(runs)

    # --- the K timed steps (median of three timed runs of all K) ---
    step_ms_total = timed(step, args.steps)
    ms_per_step = step_ms_total / args.steps
    # --- the decode kernel alone (graph of back-to-back launches) ---
    dec_ms = timed(decode_only, args.steps) / args.steps

    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()

    eb = 2
    step_bytes = wl.decode_bytes(cfg, ctx)
    append_bytes = cfg.batch * cfg.hkv * cfg.head_dim * 2 * eb
    dec_bytes = step_bytes - append_bytes
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = dec_bytes / (dec_ms * 1e-3) / 1e9

    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            tr = json.load(f)
        if tr.get("workload") == args.workload and tr.get("split_tokens", 0) == args.split_tokens:
            traffic = profile_value(TRAFFIC_FILE, "hbm_bytes_per_launch")

    fl = floors(lib, torch, cfg, inp, max_ctx, L, dec_bytes)
    del inp, qkv, kp, vp
    torch.cuda.empty_cache()

    prefill = None if args.no_prefill else prefill_bench(lib, torch)
    sampling = None if args.no_prefill else sampling_bench(lib, torch)
    model = None if args.no_model else model_bench(lib, torch)
    long_ctx = None
    if not args.no_long_context:
        long_ctx = [long_context_bench(lib, torch, n, args.seed, split_tokens=st)
                    for n, st in (("batch64_long", 0), ("batch64_long", 512), ("batch8_32k", 0))]

    cpu = None
    if not args.no_cpu_baseline:
        threads, nproc, affinity = cpu_share()
        cb = cpu_baseline(cfg, args.seed, threads=threads)
        cpu_bytes = wl.decode_bytes(cfg, cb["ctx"])
        cpu = {"value": round(cpu_bytes / cb["t"] / 1e9, 3), "unit": "GB/s",
               "cores": cb["threads"], "kind": "port", "nproc": nproc, "affinity_cpus": affinity,
               "sample": (f"one full layer step of {cfg.name} (B={cfg.batch}, RoPE + append + "
                          f"attention of every sequence), oracle C restatement with OpenMP on "
                          f"{cb['threads']} threads (the process's CPU share: {affinity} CPUs in "
                          f"its affinity mask of {nproc}, OMP_NUM_THREADS "
                          f"{os.environ.get('OMP_NUM_THREADS', 'unset')}), median of {cb['reps']} "
                          f"runs, {cb['t'] * 1e3:.1f} ms/step")}
        if cb["threads"] > 1:
            c1 = cpu_baseline(cfg, args.seed, budget_s=8.0, threads=1)
            cpu["single_core"] = {"value": round(cpu_bytes / c1["t"] / 1e9, 3), "unit": "GB/s",
                                  "cores": 1, "sample": (f"the same step on one thread, median of "
                                                         f"{c1['reps']} runs, "
                                                         f"{c1['t'] * 1e3:.1f} ms/step")}
        c1cfg = wl.CONFIGS["single_512"]
        s_all = cpu_baseline(c1cfg, args.seed, budget_s=3.0, threads=threads)
        s_one = cpu_baseline(c1cfg, args.seed, budget_s=3.0, threads=1)
        s_bytes = wl.decode_bytes(c1cfg, s_all["ctx"])
        cpu["single_512"] = {
            "workload": "single_512 (B=1, 14q/2kv, d=64, fp16, ctx 512, permuted table)",
            "us_per_step": round(s_all["t"] * 1e6, 1), "value": round(s_bytes / s_all["t"] / 1e9, 3),
            "unit": "GB/s", "cores": s_all["threads"],
            "single_core_us_per_step": round(s_one["t"] * 1e6, 1),
            "single_core_value": round(s_bytes / s_one["t"] / 1e9, 3),
            "sample": f"median of {s_all['reps']} / {s_one['reps']} runs"}

    res = {
        "metric": "paged decode attn: µs/step + achieved HBM GB/s (% peak) at B=32, 1 MI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "us_per_step": round(ms_per_step * 1e3, 3),
        "pct_of_peak_hbm": round(100 * value / PEAK_HBM_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic (seeded N(0,1)*sigma pools and queries, shuffled page allocation)",
        "config": {"workload": cfg.name, "batch": cfg.batch, "q_heads": cfg.hq,
                   "kv_heads": cfg.hkv, "head_dim": cfg.head_dim,
                   "ctx": f"U{{{cfg.ctx_lo}..{cfg.ctx_hi}}}", "mean_ctx": float(np.mean(ctx)),
                   "page_size": 16, "pool_pages": cfg.pool_pages,
                   "layers_rotated": min(L, args.steps),
                   "step": "luc_decode_step: rope + append + split-K decode with in-kernel LSE merge (one launch, one layer)",
                   "bytes_per_step": int(step_bytes),
                   "launch": "eager" if args.eager else "hip graph",
                   "split_tokens": args.split_tokens or "auto"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": traffic, "kernel": "luc_paged_decode (luc_decode_*, merge in the last split)",
                     "us_per_launch": round(dec_ms * 1e3, 3),
                     "algorithmic_bytes_per_launch": int(dec_bytes), **fl},
        "cpu_baseline": cpu,
        "code_objects": {n: (code_object_sha256(n) or "")[:16] for n in
                         ("paged_decode", "paged_prefill", "rope_append")},
        "long_context": long_ctx,
        "prefill": prefill,
        "sampling": sampling,
        "model": model,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
