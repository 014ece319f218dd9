"""Benchmark: compressed-KV scan GB/s (% HBM peak) + us/decode-step at ctx 32k, 1 GPU.

Workload: one Llama-3.2-1B-shape layer (32 query heads,
8 KV heads, d=64, 4-bit keys / 2-bit values), batch 1. Each cache is filled by
32,767 GPU appends of seeded synthetic q/k/v (insitu_amd/workload.py); every
timed step is then the configuration's one decode step from the wire: rotate
q/k/v, append the token's compressed k/v row (row 32,767), attend over all
32,768 rows, Q16 out. The scan bytes are the compressed-cache bytes the attend
reads: 8 KV heads x 32,768 rows x 52 B = 13,631,488 B.

Defeating the 256 MB Infinity Cache: the steps of the whole run (warmup, the
K steps of `value`, the 64 event-timed steps of the roofline, the two-pass line)
take caches in one rotation over 64 caches of ~13.6 MB: step i reads cache
i % 64, so between two reads of a cache the other 63 are read (a reuse distance
of ~1 GB, four times the Infinity Cache). Before each pass every cache is rewound
to 32,767 rows (a length reset, outside the timed region), so every timed step is
at ctx 32,768.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode online]
    python bench.py --copy-calibration      # a plain copy kernel of known size
    python bench.py --config c3|c4          # the larger configurations, attend only
    python bench.py --config c1             # config 1 in full, every step checked
    python bench.py --config prefill        # a 4,096-token prompt through one layer
    python bench.py --config block          # hidden states in, hidden states out, ctx 32k
    python bench.py --config probe          # bytes-only read of the C2 scan size: the launch ceiling
    python bench.py --config short          # ctx 100 in a 131,072-token cache vs a 256-token one
    python bench.py --config append         # the write path: 32,767 wire rows into an empty cache
    python bench.py --config formats        # decode steps with 8 query heads 3b/2b and 2 query heads 4b/2b

C3: batch 64, one layer, per-sequence contexts uniform in
[1024, 8192] from seed 3, each sequence its own seeded k/v and query, one
attend launch over the whole batch; 3 caches (more than the 256 MB Infinity
Cache in total) rotate between steps; every group of the last timed launch is
checked against the oracle.
C1: all 16 layers of a Llama-3.2-1B-shape block, batch 1,
4,096 sequential decode steps from an empty cache, each step one insitu_step
(rotate, append, attend) per layer; layer l draws its q/k/v from its own
seeded stream (seed 1000 + l, as config 0). Every step of every layer is then
compared with the oracle's online softmax over rows 0 .. t, and every cache
byte with the oracle's packed rows. It is a parity run with its timing, not
the headline line.
C4: Llama-3-8B shape (32 query heads, 8 KV heads, d=128,
3-bit K and V), batch 16, ctx 131,072, 32 layers: one step is the 32 layers'
attends, over a 53.7 GB resident cache. Every sequence of every layer has its
own k/v (drawn on the GPU, seeded, 1% outlier channels x16) and query; the last
timed launch is checked against the oracle on two KV heads of every sequence.
Block: the whole attention block per decode token (AttentionBlock.forward,
kernel.py:177-357): fp16 q/k/v projections, attention scale, RoPE and the cast
to the wire, rotate, append, attend over ctx 32,768, to_float and W_o', with
seeded random fp16 weights; 20 blocks (weights and caches, more than the
Infinity Cache in total) rotate between steps.
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

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, published
CTX = 32768
N_Q, N_KV, D = 32, 8, 64
ROW = 52
N_CU = 256                 # MI355X compute units


def rotate_q(q_wire):
    """The query row rotated as the step rotates it (rotate.py:170-197), for the oracle."""
    from oracle.rotate import rotate, signs_from_seed
    return rotate(np.asarray(q_wire).astype(np.int64), signs_from_seed(D, 0, 1))


def _args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--mode", default="online", choices=["online", "two_pass", "split", "serial"])
    ap.add_argument("--chunk-tokens", type=int, default=0, choices=[0, 512, 1024],
                    help="tokens per chunk of the chunked attend for C2/C3/C4 (0: the cache default, 1,024)")
    ap.add_argument("--kernel", default="auto", choices=["auto", "step", "chunked"],
                    help="the decode step's kernel (C2, short): the automatic choice, the step kernel "
                         "(attend_step.hip) or the chunked attend's fused step")
    ap.add_argument("--caches", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=CTX)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--config", default="c2",
                    choices=["c1", "c2", "c3", "c4", "prefill", "block", "probe", "short", "append", "formats"])
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--c1-layers", type=int, default=16)
    ap.add_argument("--c1-steps", type=int, default=4096)
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "step_kernel_c2_traffic.json")


# The kernels insitu_step launches for one decode step, per mode, at C2's format
# (d = 64, 4-bit keys, 2-bit values, 4 query heads per KV head): online and split
# mode are one launch of the step kernel (attend_step.hip), or of the chunked
# attend's fused step when --kernel chunked pins it.
STEP_KERNEL = {
    "online": "insitu::stepk::step_kernel<4, 2>",
    "split": "insitu::stepk::step_kernel<4, 2>",
    "two_pass": "insitu::step_write_kernel + insitu::chunk_max_kernel + insitu::chunk_kernel",
    "serial": "insitu::step_write_kernel + insitu::attend_serial_kernel",
}
CHUNKED_STEP_KERNEL = "insitu::chunk_kernel<64, 4, true, false, true>"
TIMED_LAUNCHES = 64        # event-timed attends behind the roofline median (at least 50)


def measured_traffic(kernel: str, ctx: int):
    """HBM bytes per attend launch from the committed FETCH_SIZE/WRITE_SIZE passes,
    and where they come from.

    The passes profile one kernel at ctx 32,768; for another kernel or context there
    is no measurement, and the field is null.
    """
    if ctx != CTX or not os.path.exists(TRAFFIC_FILE):
        return None, None
    with open(TRAFFIC_FILE) as f:
        t = json.load(f)
    if t.get("kernel") != kernel:
        return None, f"none for {kernel} ({os.path.relpath(TRAFFIC_FILE, ROOT)} covers {t.get('kernel')})"
    return t.get("traffic_bytes"), (f"{os.path.relpath(TRAFFIC_FILE, ROOT)}: rocprofv3 FETCH_SIZE + WRITE_SIZE "
                                    f"per dispatch, each scaled by a plain copy's counters")


def copy_calibration() -> None:
    """A plain device copy of known size, for scaling FETCH_SIZE/WRITE_SIZE counters."""
    import torch
    n = 256 << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_dispatch": n, "dispatches": 5}))


def cpu_baseline(cache, q_rot_all, out_gpu, wire, budget_s: float = 20.0):
    """The oracle's numpy restatement of the decode step, timed on this box's host cores
    (the reference's CPU path for the step): rotate the step's q/k/v, encode and pack its k/v row, then
    attend_online (the per-token loop, the parity golden) on the step's cache, KV group
    by KV group within `budget_s` (at least one group; the GPU output of every timed
    group is checked bit for bit), and the vectorized attend_two_pass on every group.
    Also a whole C0 step (ctx 512) timed end to end."""
    from oracle.attention import attend_online, attend_two_pass
    from oracle.quantize import Cache, Format, encode, pack
    from oracle.rotate import rotate, signs_from_seed
    from insitu_amd.workload import Workload
    fmt = Format()
    sg = signs_from_seed(D, 0, 1)
    qw, kw, vw = (np.asarray(x, dtype=np.int64) for x in wire)
    t0 = time.perf_counter()
    qr = rotate(qw.reshape(-1, D), sg)
    kr = rotate(kw.reshape(-1, D), sg)
    vr = rotate(vw.reshape(-1, D), sg)
    t_rot = time.perf_counter() - t0
    t0 = time.perf_counter()
    rows = [pack(encode(kr[h][None], vr[h][None], fmt), fmt) for h in range(N_KV)]
    t_enc = time.perf_counter() - t0
    if not np.array_equal(qr, q_rot_all):
        raise AssertionError("the oracle's rotation of the step's query differs from the GPU's")
    kvs = [cache.view(h).host() for h in range(N_KV)]
    n = kvs[0].k_idx.shape[0]
    for h in range(N_KV):
        if not np.array_equal(cache.read_rows(h, n - 1, 1), rows[h]):
            raise AssertionError(f"the step's row of KV head {h} differs from the oracle's encode + pack")
    rows_t, done, t_on = 0, 0, 0.0
    for h in range(N_KV):
        q = q_rot_all[4 * h:4 * h + 4]
        t0 = time.perf_counter()
        want, _ = attend_online(q, kvs[h], fmt)
        t_on += time.perf_counter() - t0
        if not np.array_equal(want, out_gpu[4 * h:4 * h + 4]):
            raise AssertionError(f"bench step disagrees with the oracle on KV group {h}")
        rows_t += kvs[h].k_idx.shape[0]
        done += 1
        if t_on > budget_s:
            break
    t0 = time.perf_counter()
    for h in range(N_KV):
        attend_two_pass(q_rot_all[4 * h:4 * h + 4], kvs[h], fmt)
    t_two = time.perf_counter() - t0
    # C0: one decode step at ctx 512 (the token attends to itself), end to end
    q0, k0, v0 = (x[0] for x in Workload(seed=0).steps(512))
    host = Cache(N_KV, 512, fmt)
    host.append_rotated(rotate(k0[:511].reshape(-1, D), sg).reshape(511, N_KV, D),
                        rotate(v0[:511].reshape(-1, D), sg).reshape(511, N_KV, D))
    t0 = time.perf_counter()
    qs = rotate(q0[511].reshape(-1, D), sg)
    host.append_rotated(rotate(k0[511].reshape(-1, D), sg)[None], rotate(v0[511].reshape(-1, D), sg)[None])
    for h in range(N_KV):
        attend_online(qs[4 * h:4 * h + 4], host.view(h), fmt)
    t_c0 = time.perf_counter() - t0
    gbs = rows_t * ROW / t_on / 1e9
    per_group = t_on / done
    env = {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")}
    return {"value": round(gbs, 6), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle numpy attend_online (per-token loop) on {done} of {N_KV} KV groups "
                      f"of the last timed step's cache ({int(rows_t)} rows, {t_on:.1f} s)",
            "affinity_cores": len(os.sched_getaffinity(0)), "thread_env": env,
            "threads_used": "1 (a Python loop; int64 einsum has no BLAS path)",
            "s_rotate_step": round(t_rot, 5), "s_encode_pack_step": round(t_enc, 5),
            "s_attend_online_per_kv_group": round(per_group, 3),
            "s_attend_two_pass_all_groups": round(t_two, 3),
            "s_per_decode_step_c2_extrapolated": round(t_rot + t_enc + per_group * N_KV, 3),
            "s_per_decode_step_c0_measured": round(t_c0, 4)}


def _timed_each(ctx, launch, reps: int):
    """Per-launch kernel times (us) of `reps` calls of launch(i), from HIP events attached to
    the dispatches on the library's stream (insitu_ctx_timing_read_each)."""
    import ctypes
    from insitu_amd import _lib
    lib = ctx.lib
    _lib.check(lib.insitu_ctx_timing(ctx.handle, 1))
    for i in range(reps):
        launch(i)
    ms = (ctypes.c_double * reps)()
    n = ctypes.c_int64()
    _lib.check(lib.insitu_ctx_timing_read_each(ctx.handle, ms, reps, ctypes.byref(n)))
    _lib.check(lib.insitu_ctx_timing(ctx.handle, 0))
    if n.value != reps:
        raise RuntimeError(f"timed {n.value} launches of {reps}")
    return np.array(ms[:reps]) * 1e3


def bench_probe(a) -> int:
    """The ceiling of one launch: a bytes-only read of the C2 scan size (13,631,488 B) at
    several grid shapes, rotating over 40 buffers (545 MB, more than twice the 256 MB
    Infinity Cache), and an empty launch. No attention work; the analogue of the
    reference's DDR probe (rtl/ddr_probe.sv)."""
    import torch

    from insitu_amd import _lib
    from insitu_amd.runtime import default_context, ptr

    ctx = default_context(0)
    lib = ctx.lib
    nbytes = N_KV * CTX * ROW
    nbuf = 40
    g = torch.Generator(device=ctx.torch_device).manual_seed(0)
    bufs = [torch.randint(0, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, device=ctx.torch_device,
                          generator=g) for _ in range(nbuf)]
    sink = torch.zeros(256, dtype=torch.int32, device=ctx.torch_device)
    reps = max(a.steps, 50)
    rows = []
    for layout in (0, 1):
        for n_wg in (256, 512, 1024, 2048, 4096):
            def launch(i, layout=layout, n_wg=n_wg):
                _lib.check(lib.insitu_probe_read(ctx.handle, ptr(bufs[i % nbuf]), nbytes, n_wg, layout,
                                                 ptr(sink)))
            for i in range(a.warmup):
                launch(i)
            torch.cuda.synchronize()
            us = _timed_each(ctx, launch, reps)
            med = float(np.median(us))
            rows.append({"kernel": "probe_read_kernel", "layout": ["grid-stride", "span per workgroup"][layout],
                         "workgroups": n_wg, "median_us": round(med, 3), "min_us": round(float(us.min()), 3),
                         "gbs_median": round(nbytes / med / 1e3, 1)})
            print(f"probe: layout {layout} wg {n_wg}: {med:.2f} us", file=sys.stderr, flush=True)
    # the same buffer every time: what a launch reads when the bytes sit in the Infinity Cache
    def launch_hot(i):
        _lib.check(lib.insitu_probe_read(ctx.handle, ptr(bufs[0]), nbytes, 1024, 0, ptr(sink)))
    for i in range(a.warmup):
        launch_hot(i)
    us = _timed_each(ctx, launch_hot, reps)
    rows.append({"kernel": "probe_read_kernel", "layout": "grid-stride, one buffer (Infinity Cache resident)",
                 "workgroups": 1024, "median_us": round(float(np.median(us)), 3),
                 "gbs_median": round(nbytes / float(np.median(us)) / 1e3, 1)})
    for n_wg in (256, 1024):
        def launch_empty(i, n_wg=n_wg):
            _lib.check(lib.insitu_probe_empty(ctx.handle, n_wg, ptr(sink)))
        for i in range(a.warmup):
            launch_empty(i)
        us = _timed_each(ctx, launch_empty, reps)
        rows.append({"kernel": "probe_empty_kernel", "workgroups": n_wg,
                     "median_us": round(float(np.median(us)), 3)})
    best = min((r for r in rows if r["kernel"] == "probe_read_kernel" and "one buffer" not in r["layout"]),
               key=lambda r: r["median_us"])
    res = {"metric": "bytes-only HBM read of the C2 scan size in one launch (the single-launch ceiling)",
           "value": best["gbs_median"], "unit": "GB/s", "n_gpus": 1, "steps": reps, "warmup": a.warmup,
           "higher_is_better": True, "dtype": "u8", "data": "random bytes",
           "config": {"workload": f"read {nbytes} B per launch, {nbuf} rotating buffers "
                                  f"({nbuf * nbytes / 2 ** 20:.0f} MiB)"},
           "frac_of_peak": round(best["gbs_median"] / HBM_PEAK_GBS, 4), "rows": rows}
    print(json.dumps(res))
    return 0


def _check_groups(cache, out, q, groups, fmt, G=4):
    """The checker leg of C3/C4: oracle/c's attend_online over the device's own rows for
    each (sequence, KV head) in groups, against `out` (batch, n_q, d). The rows are read
    on this thread; decoding and the oracle run in threads. Returns the groups that differ."""
    import concurrent.futures

    from insitu_amd.cache import unpack_rows
    from oracle import native
    rows = {bh: cache.read_rows(bh[1], 0, None, bh[0]) for bh in groups}
    kb, vb = cache.quant.key_bits, cache.quant.value_bits

    def check(bh):
        b, h = bh
        kv = unpack_rows(rows[bh], cache.head_dim, kb, vb)
        want, _ = native.attend_online(q[b, G * h:G * (h + 1)], kv, fmt)
        return bh, bool(np.array_equal(out[b, G * h:G * (h + 1)], want))

    workers = max(1, min(16, len(os.sched_getaffinity(0))))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:
        return [bh for bh, ok in ex.map(check, groups) if not ok]


def bench_scale(a) -> int:
    """C3 / C4: the attend launches alone, over caches filled by GPU appends, each
    sequence with its own seeded k/v and query; the last timed launch checked against
    the oracle."""
    import torch

    from insitu_amd import QuantConfig
    from insitu_amd.attention import CompressedAttention
    from insitu_amd.cache import CompressedCache
    from insitu_amd.rotate import Rotation
    from insitu_amd.runtime import default_context
    from insitu_amd.workload import fill_on_device, fill_ragged
    from oracle.quantize import Format

    ctx = default_context(0)
    if a.config == "c3":
        d, kb, vb, batch, n_caches, row = 64, 4, 2, 64, 3, 52
        lens = np.random.default_rng(3).integers(1024, 8193, size=batch)
        workload = ("C3: Llama-3.2-1B-shape single layer, batch 64, ragged contexts "
                    "uniform in [1024, 8192] (seed 3), 4b K / 2b V, one attend launch")
        data = ("synthetic: per sequence b of cache i, Workload(seed=3000 + 100 i + b) k/v "
                "(N(0,1), 4 outlier channels x8 per head, Q8.16) and one query row per head")
    else:
        d, kb, vb, batch, n_caches, row = 128, 3, 3, 16, 32, 100
        lens = np.full(batch, 131072)
        workload = ("C4: Llama-3-8B shape (32 q heads, 8 KV heads, d=128), 3b K / 3b V, "
                    "batch 16, ctx 131072, 32 layers (one step = 32 attend launches)")
        data = ("synthetic, drawn on the GPU: per layer i and sequence b, torch.Generator seed "
                "4000 + 100 i + b, N(0,1) k/v with 1% of channels per head x16, Q8.16; one query "
                "row per head per sequence")
    quant = QuantConfig(key_bits=kb, value_bits=vb)
    fmt = Format(d=d, key_bits=kb, value_bits=vb)
    rot = Rotation.for_quant(quant, d)
    caches = [CompressedCache(N_KV, d, int(lens.max()), quant, batch=batch, n_q_heads=N_Q,
                              chunk_tokens=a.chunk_tokens, ctx=ctx)
              for _ in range(n_caches)]
    t_fill = time.perf_counter()
    qs = []
    for i, c in enumerate(caches):
        if a.config == "c3":
            q, _ = fill_ragged(c, lens, 3000 + 100 * i, rot, ctx)
        else:
            q, _ = fill_on_device(c, int(lens[0]), 4000 + 100 * i, rot, ctx)
        qs.append(q)
        torch.cuda.synchronize()
        print(f"{a.config}: cache {i + 1} of {n_caches} filled", file=sys.stderr, flush=True)
    t_fill = time.perf_counter() - t_fill
    qd = [ctx.to_device(q, torch.int32) for q in qs]
    attn = [CompressedAttention(c) for c in caches]
    outs = [torch.empty((batch, N_Q, d), dtype=torch.int32, device=ctx.torch_device) for _ in caches]
    step_bytes = float(N_KV * row * lens.sum()) * (n_caches if a.config == "c4" else 1)
    last = {"cache": 0}

    def step(i):
        if a.config == "c4":
            for l, at in enumerate(attn):
                at.attend(qd[l], a.mode, out=outs[l], stats=False)
            last["cache"] = n_caches - 1
        else:
            j = i % n_caches
            attn[j].attend(qd[j], a.mode, out=outs[j], stats=False)
            last["cache"] = j

    import ctypes
    from insitu_amd import _lib
    lib = ctx.lib
    n_launch = a.steps * (n_caches if a.config == "c4" else 1)
    for i in range(a.warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _lib.check(lib.insitu_ctx_timing(ctx.handle, 1))
    t0 = time.perf_counter()
    e0.record()
    for i in range(a.steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = (ctypes.c_double * n_launch)()
    n_att = ctypes.c_int64()
    _lib.check(lib.insitu_ctx_timing_read_each(ctx.handle, ms, n_launch, ctypes.byref(n_att)))
    _lib.check(lib.insitu_ctx_timing(ctx.handle, 0))
    us_each = np.array(ms[:n_att.value]) * 1e3
    ev_s = e0.elapsed_time(e1) / 1e3          # the launches with their query staging
    kern_s = us_each.sum() / 1e6              # the attend kernels alone
    per_launch = step_bytes / (n_caches if a.config == "c4" else 1)
    us_med = float(np.median(us_each))
    # the checker leg: the last timed launch's output against the oracle on the device's rows
    j = last["cache"]
    out = outs[j].cpu().numpy()
    if a.config == "c3":
        groups = [(b, h) for b in range(batch) for h in range(N_KV)]
    else:
        groups = [(b, h) for b in range(batch) for h in (0, 5)]
    t_chk = time.perf_counter()
    bad = _check_groups(caches[j], out, qs[j], groups, fmt)
    t_chk = time.perf_counter() - t_chk
    gbs = per_launch / (us_med * 1e-6) / 1e9
    res = {
        "metric": "compressed-KV scan GB/s (% HBM peak)",
        "value": round(step_bytes * a.steps / wall / 1e9, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(wall / a.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int64",
        "data": data,
        "config": {"workload": workload, "mode": a.mode, "chunk_tokens": a.chunk_tokens or 1024, "batch": batch,
                   "ctx_total": int(lens.sum()), "ctx_min": int(lens.min()), "ctx_max": int(lens.max()),
                   "caches": n_caches, "head_dim": d, "row_bytes": row,
                   "resident_gb": round(sum(c.layout()["device_total_bytes"] for c in caches) / 1e9, 2),
                   "fill_s": round(t_fill, 1)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 5), "traffic": None,
                     "kernel": "insitu::chunk_kernel (sequential, d = %d)" % d,
                     "algorithmic_bytes_per_launch": per_launch,
                     "attend_us_median": round(us_med, 3), "attend_us_mean": round(float(us_each.mean()), 3),
                     "launches_timed": int(n_att.value),
                     "us_per_step_kernels": round(kern_s / a.steps * 1e6, 2),
                     "us_per_step_events_with_query_prep": round(ev_s / a.steps * 1e6, 2)},
        "cpu_baseline": None,
        "checked": {"launch": f"the last timed launch (cache {j})", "groups": len(groups),
                    "mismatched": [list(g) for g in bad], "oracle": "oracle/c attend_online on the "
                    "device's rows", "check_s": round(t_chk, 1)},
    }
    print(json.dumps(res))
    return 0 if not bad else 1


def bench_append(a) -> int:
    """The write path at C2's shape: 32,767 wire rows (8 KV heads, d=64, 4b/2b) into an empty
    cache, (1) rotated by two rotate launches then appended (append_rotated), (2) rotated and
    appended in one launch (append_wire, kernel.py:271-272 + :283-284). Times from HIP events
    on the library's stream around each call, median of the repetitions; the two paths' rows
    are compared byte for byte."""
    import torch

    from insitu_amd import QuantConfig
    from insitu_amd.cache import CompressedCache
    from insitu_amd.rotate import Rotation
    from insitu_amd.runtime import default_context
    from insitu_amd.workload import Workload

    ctx = default_context(0)
    quant = QuantConfig(key_bits=4, value_bits=2)
    rot = Rotation.for_quant(quant, D)
    n = CTX - 1
    wl = Workload(seed=0)
    _, k, v = wl.steps(n)
    kd = ctx.to_device(k[0], torch.int32)
    vd = ctx.to_device(v[0], torch.int32)
    sp = ctx.lib.insitu_ctx_stream(ctx.handle)          # None: the null stream
    stream = torch.cuda.ExternalStream(int(sp)) if sp else torch.cuda.default_stream()
    reps = max(a.steps, 20)

    def timed(c, fn):
        us = []
        for i in range(reps + 2):
            c.set_length(0)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            e1.synchronize()
            if i >= 2:
                us.append(e0.elapsed_time(e1) * 1e3)
        return np.array(us)

    a_c = CompressedCache(N_KV, D, CTX, quant, n_q_heads=N_Q, ctx=ctx)
    b_c = CompressedCache(N_KV, D, CTX, quant, n_q_heads=N_Q, ctx=ctx)
    us_two = timed(a_c, lambda: a_c.append_rotated(rot.apply(kd, ctx), rot.apply(vd, ctx)))
    us_one = timed(b_c, lambda: b_c.append_wire(kd, vd))
    for h in (0, N_KV - 1):
        if not np.array_equal(a_c.read_rows(h, 0, n), b_c.read_rows(h, 0, n)):
            raise AssertionError("append_wire and rotate + append_rotated wrote different rows")
    moved = n * N_KV * (2 * D * 4 + ROW)         # int32 k and v in, packed rows out
    res = {
        "metric": "write path: rows appended per second, C2 shape",
        "value": round(n * N_KV / (np.median(us_one) * 1e-6) / 1e6, 2), "unit": "M rows/s",
        "n_gpus": 1, "steps": reps, "higher_is_better": True, "dtype": "int64",
        "data": "synthetic (seeded N(0,1) k/v with 4 outlier channels x8 per head, Q8.16)",
        "config": {"workload": f"{n} tokens x {N_KV} KV heads, d={D}, 4b K / 2b V, into an empty cache"},
        "append_wire_us_median": round(float(np.median(us_one)), 2),
        "append_wire_us_min": round(float(us_one.min()), 2),
        "rotate_then_append_us_median": round(float(np.median(us_two)), 2),
        "append_wire_GBps": round(moved / (np.median(us_one) * 1e-6) / 1e9, 1),
        "checked": "append_wire rows equal rotate + append_rotated rows (KV heads 0 and 7)",
    }
    print(json.dumps(res))
    return 0


def bench_formats(a) -> int:
    """Decode steps in formats outside C2's: the reference's default 3-bit keys with 8 query
    heads a KV head (TinyLlama's group, config.py:122-125, 141), and 2 query heads a KV head
    with 4-bit keys, each at ctx 9,000 (8 KV heads, d=64, 2-bit values): per-launch event
    times of the attend over 50 steps, the statistics' serial fallbacks (0: every head on
    the fast path), and the last step checked against the oracle."""
    import torch

    from insitu_amd import QuantConfig, _lib
    from insitu_amd.cache import CompressedCache
    from insitu_amd.runtime import default_context, ptr
    from oracle import native
    from oracle.quantize import Cache, Format

    ctx = default_context(0)
    lib = ctx.lib
    rng = np.random.default_rng(9)
    T0, reps = 9000, max(a.steps, 50)
    lines = {}
    for name, G, kb in (("G8_3b2b", 8, 3), ("G2_4b2b", 2, 4)):
        quant = QuantConfig(key_bits=kb, value_bits=2)
        f = Format(key_bits=kb, value_bits=2)
        n_q = N_KV * G
        # N(0, 1) rows in Q8.16, the wire's format (the prompt's rows rotated as a step would)
        def wire(*shape):
            return np.rint(rng.standard_normal(shape) * 65536.0).astype(np.int64)
        sg = __import__("oracle.rotate", fromlist=["signs_from_seed"]).signs_from_seed(D, 0, 1)
        rot = __import__("oracle.rotate", fromlist=["rotate"]).rotate
        kr = rot(wire(T0 * N_KV, D), sg).reshape(T0, N_KV, D)
        vr = rot(wire(T0 * N_KV, D), sg).reshape(T0, N_KV, D)
        c = CompressedCache(N_KV, D, T0 + reps + a.warmup, quant, n_q_heads=n_q, ctx=ctx)
        c.append_rotated(kr, vr)
        qw = ctx.to_device(wire(reps + a.warmup, n_q, D), torch.int32)
        kw = ctx.to_device(wire(reps + a.warmup, N_KV, D), torch.int32)
        vw = ctx.to_device(wire(reps + a.warmup, N_KV, D), torch.int32)
        out = torch.empty((n_q, D), dtype=torch.int32, device=ctx.torch_device)
        st = _lib.Stats()
        serial = 0

        def launch(i):
            nonlocal serial
            _lib.check(lib.insitu_step(c.handle, ptr(qw[i]), ptr(kw[i]), ptr(vw[i]), ptr(out), 0, st))
            serial += st.serial_fallbacks

        for i in range(a.warmup):
            launch(i)
        c.set_length(T0)
        us = _timed_each(ctx, lambda i: launch(a.warmup + i), reps)
        # the last step against the oracle over the cache's rows
        q_last = rotate_q(qw[a.warmup + reps - 1].cpu().numpy())
        want = np.concatenate([native.attend_online(q_last[G * h:G * h + G], c.view(h), f)[0]
                               for h in range(N_KV)])
        if not np.array_equal(want, out.cpu().numpy().astype(np.int64).reshape(-1, D)):
            raise AssertionError(f"{name}: the last step disagrees with the oracle")
        lines[name] = {"query_heads_per_kv_head": G, "key_bits": kb, "value_bits": 2,
                       "ctx_first": T0 + 1, "attend_us_median": round(float(np.median(us)), 3),
                       "attend_us_min": round(float(us.min()), 3), "serial_fallbacks": int(serial),
                       "GB/s": round(N_KV * c.layout()["row_bytes"] * (T0 + reps // 2) /
                                     (np.median(us) * 1e-6) / 1e9, 1)}
    res = {"metric": "decode step (rotate + append + attend) in other formats: attend us",
           "value": lines["G8_3b2b"]["attend_us_median"], "unit": "us", "n_gpus": 1, "steps": reps,
           "higher_is_better": False, "dtype": "int64", "data": "synthetic (seeded N(0,1) q/k/v, Q8.16)",
           "config": {"workload": "8 KV heads, d=64, ctx 9,000 on, batch 1"}, "formats": lines,
           "checked": "the last step of each format equal to oracle/c attend_online"}
    print(json.dumps(res))
    return 0


def bench_short(a) -> int:
    """Decode at a short context in a large cache: ctx 100 (C2's format) in caches sized for
    131,072 tokens and for 256, the same steps on each, per-launch event times. The attend
    grid follows the longest sequence, so the capacity costs nothing."""
    import torch

    from insitu_amd import QuantConfig, _lib
    from insitu_amd.cache import CompressedCache
    from insitu_amd.rotate import Rotation
    from insitu_amd.runtime import default_context, ptr
    from insitu_amd.workload import Workload

    ctx = default_context(0)
    quant = QuantConfig(key_bits=4, value_bits=2)
    rot = Rotation.for_quant(quant, D)
    n0 = 99
    wl = Workload(seed=0)
    _, k, v = wl.steps(n0)
    kr, vr = rot.apply(k[0], ctx), rot.apply(v[0], ctx)
    reps = max(a.steps, 50)
    q, kw, vw = (ctx.to_device(x[0], torch.int32) for x in wl.steps(reps))
    out = torch.empty((N_Q, D), dtype=torch.int32, device=ctx.torch_device)
    lib = ctx.lib
    res_caps = {}
    for cap in (131072, 256):
        c = CompressedCache(N_KV, D, cap, quant, n_q_heads=N_Q, ctx=ctx)
        c.append_rotated(kr, vr)
        if a.kernel != "auto":
            c.pin_kernel(a.kernel)

        def launch(i, c=c):
            _lib.check(lib.insitu_step(c.handle, ptr(q[i]), ptr(kw[i]), ptr(vw[i]), ptr(out),
                                       _lib.MODES[a.mode], None))

        for i in range(a.warmup):
            launch(i)
        c.set_length(n0)                       # the timed steps start at ctx n0 + 1 again
        us = _timed_each(ctx, launch, reps)
        res_caps[cap] = {"attend_us_median": round(float(np.median(us)), 3),
                         "attend_us_min": round(float(us.min()), 3), "ctx_first": n0 + 1,
                         "ctx_last": n0 + reps}
    res = {
        "metric": "decode step at a short context: attend us by cache capacity",
        "value": res_caps[131072]["attend_us_median"], "unit": "us", "n_gpus": 1, "steps": reps,
        "higher_is_better": False, "dtype": "int64",
        "data": "synthetic (seeded N(0,1) q/k/v with 4 outlier channels x8 per head, Q8.16)",
        "config": {"workload": "C2's format (8 KV heads, d=64, 4b/2b), batch 1, insitu_step from "
                               f"ctx {n0 + 1} on, caches of capacity 131,072 and 256", "mode": a.mode},
        "by_capacity": res_caps,
    }
    print(json.dumps(res))
    return 0


def bench_c1(a) -> int:
    """Config 1 in full: 16 layers x 4,096 decode steps from empty, every step checked."""
    import concurrent.futures
    import ctypes

    import torch

    from insitu_amd import QuantConfig, _lib
    from insitu_amd.cache import CompressedCache
    from insitu_amd.runtime import default_context, ptr
    from insitu_amd.workload import Workload
    from oracle import native
    from oracle.quantize import Format, encode, pack
    from oracle.rotate import rotate, signs_from_seed

    L, S = a.c1_layers, a.c1_steps
    ctx = default_context(0)
    quant = QuantConfig(key_bits=4, value_bits=2)
    fmt = Format()
    wire = [Workload(seed=1000 + l).steps(S) for l in range(L)]
    caches = [CompressedCache(N_KV, D, S, quant, batch=1, n_q_heads=N_Q, ctx=ctx) for _ in range(L)]
    dev = [tuple(ctx.to_device(x[0], torch.int32) for x in w) for w in wire]
    outs = torch.empty((L, S, N_Q, D), dtype=torch.int32, device=ctx.torch_device)
    lib = ctx.lib
    mode = _lib.MODES[a.mode]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(S):
        for l in range(L):
            qd, kd, vd = dev[l]
            _lib.check(lib.insitu_step(caches[l].handle, ptr(qd[t]), ptr(kd[t]), ptr(vd[t]),
                                       ptr(outs[l, t]), mode, None))
        if t % 512 == 511:
            torch.cuda.synchronize()
            print(f"c1: {t + 1} of {S} steps on the GPU", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    gpu_s = time.perf_counter() - t0
    got = outs.cpu().numpy()
    bufs = [c.buf for c in caches]

    sg = signs_from_seed(D, 0, 1)

    def check(l):
        q, k, v = (np.asarray(x[0], dtype=np.int64) for x in wire[l])
        qr = rotate(q.reshape(-1, D), sg).reshape(S, N_Q, D)
        kr = rotate(k.reshape(-1, D), sg).reshape(S, N_KV, D)
        vr = rotate(v.reshape(-1, D), sg).reshape(S, N_KV, D)
        heads = [encode(kr[:, h], vr[:, h], fmt) for h in range(N_KV)]
        want = native.decode_steps(qr, heads, fmt)
        bad_steps = np.nonzero((got[l] != want).reshape(S, -1).any(axis=1))[0]
        rows = np.stack([pack(hd, fmt) for hd in heads], axis=1)
        return l, bad_steps, bool(np.array_equal(bufs[l][:S], rows))

    workers = max(1, min(16, len(os.sched_getaffinity(0))))
    t1 = time.perf_counter()
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:
        results = list(ex.map(check, range(L)))
    cpu_s = time.perf_counter() - t1
    mism = {l: bs[:5].tolist() for l, bs, _ in results if len(bs)}
    cache_bad = [l for l, _, ok in results if not ok]
    rows_scanned = N_KV * L * S * (S + 1) // 2
    res = {
        "metric": "config-1 parity: every decode step of every layer equal to the oracle",
        "value": int(sum(S - len(bs) for _, bs, _ in results)),
        "unit": "steps bit-exact",
        "steps_total": L * S,
        "mismatched_steps_by_layer": mism,
        "cache_bytes_mismatched_layers": cache_bad,
        "n_gpus": 1,
        "higher_is_better": True,
        "dtype": "int64",
        "data": "synthetic (seeded N(0,1) q/k/v with 4 outlier channels x8 per head, Q8.16; seed 1000 + layer)",
        "config": {"workload": f"C1: {L} Llama-3.2-1B-shape layers, batch 1, {S} sequential decode steps "
                               f"from an empty cache, insitu_step per layer and step", "mode": a.mode},
        "gpu_s": round(gpu_s, 3),
        "us_per_layer_step": round(gpu_s / (L * S) * 1e6, 2),
        "scan_gb": round(rows_scanned * ROW / 1e9, 3),
        "cpu_check_s": round(cpu_s, 1),
        "cpu_check": f"oracle/c orc_decode_steps per layer on {workers} threads",
    }
    print(json.dumps(res))
    return 0 if not mism and not cache_bad else 1


def bench_prefill(a) -> int:
    """A prompt through one Llama-3.2-1B-shape layer: rotate, append, then every
    query at once (insitu_attend_causal; query i attends rows 0 .. i)."""
    import torch

    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    from insitu_amd.runtime import default_context
    from insitu_amd.workload import Workload
    from oracle import native
    from oracle.quantize import Format, encode
    from oracle.rotate import rotate, signs_from_seed

    n = a.prompt
    ctx = default_context(0)
    q, k, v = (x[0] for x in Workload(seed=0).steps(n))
    blk = AttentionBlock(ModelConfig.llama32_1b(), QuantConfig(key_bits=4, value_bits=2),
                         capacity=n, softmax=a.mode, ctx=ctx)
    qd, kd, vd = (ctx.to_device(x, torch.int32) for x in (q, k, v))
    reps = max(1, min(a.steps, 10))
    for _ in range(max(1, a.warmup // 2)):
        blk.reset()
        blk.prefill(qd, kd, vd, stats=False)
    torch.cuda.synchronize()
    wall = 0.0
    for _ in range(reps):
        blk.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = blk.prefill(qd, kd, vd, stats=False)
        torch.cuda.synchronize()
        wall += time.perf_counter() - t0
    wall /= reps
    # spot check against the C oracle: queries 0, n/2 and n-1 of every KV group
    got = out.cpu().numpy().reshape(n, N_Q, D)
    sg = signs_from_seed(D, 0, 1)
    qr = rotate(np.asarray(q, dtype=np.int64).reshape(-1, D), sg).reshape(n, N_Q, D)
    kr = rotate(np.asarray(k, dtype=np.int64).reshape(-1, D), sg).reshape(n, N_KV, D)
    vr = rotate(np.asarray(v, dtype=np.int64).reshape(-1, D), sg).reshape(n, N_KV, D)
    fmt = Format()
    heads = [encode(kr[:, h], vr[:, h], fmt) for h in range(N_KV)]
    bad = 0
    for i in (0, n // 2, n - 1):
        if a.mode == "two_pass":
            want = np.concatenate([native.attend_two_pass(qr[i, 4 * h:4 * h + 4],
                                                          heads[h].select(slice(0, i + 1)), fmt)[0]
                                   for h in range(N_KV)])
        else:
            want = native.decode_steps(qr[i:i + 1], heads, fmt, base=i)[0]
        bad += int((got[i] != want).any())
    rows = N_KV * n * (n + 1) // 2
    res = {
        "metric": "prefill: prompt tokens per second through one layer (rotate, append, attend)",
        "value": round(n / wall, 1), "unit": "tokens/s", "n_gpus": 1, "steps": reps,
        "ms_per_prefill": round(wall * 1e3, 3), "higher_is_better": True, "dtype": "int64",
        "data": "synthetic (seeded N(0,1) q/k/v with 4 outlier channels x8 per head, Q8.16)",
        "config": {"workload": f"prefill of a {n}-token prompt, Llama-3.2-1B-shape layer, 4b K / 2b V",
                   "mode": a.mode},
        "scan_gb": round(rows * ROW / 1e9, 3),
        "effective_scan_gbs": round(rows * ROW / wall / 1e9, 1),
        "spot_check_queries_wrong": bad,
    }
    print(json.dumps(res))
    return 0 if bad == 0 else 1


LLAMA32_1B_HF = {"hidden_size": 2048, "num_attention_heads": 32, "num_key_value_heads": 8,
                 "head_dim": 64, "rope_theta": 500000.0, "max_position_embeddings": 131072,
                 "rope_scaling": {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                  "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}}


def bench_block(a) -> int:
    """One decode token through the whole block: hidden (1, 2048) float32 in,
    (1, 2048) out; the last step of the last block checked against the oracle."""
    import torch

    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.block import AttentionBlock
    from insitu_amd.host import Weights
    from insitu_amd.runtime import default_context
    from oracle import host as oh
    from oracle import native
    from oracle.quantize import Format
    from oracle.rotate import rotate, signs_from_seed

    ctx = default_context(0)
    # Llama-3.2-1B's attention shape and RoPE (theta 5e5, llama3 scaling, 131,072
    # positions): the decode tokens sit at positions 32,767 and on
    model = ModelConfig.from_hf(LLAMA32_1B_HF)
    quant = QuantConfig(key_bits=4, value_bits=2)
    n_total = a.warmup + a.steps
    per_block = (n_total + a.caches - 1) // a.caches
    wl_rng = np.random.default_rng(0)
    blocks = []
    from insitu_amd.workload import Workload
    _, kr_src, vr_src = Workload(seed=0).steps(a.ctx - 1)
    for b in range(a.caches):
        blk = AttentionBlock(model, quant, capacity=a.ctx - 1 + per_block, ctx=ctx)
        blk.weights = Weights.random(model, blk.rotation, seed=b, ctx=ctx)
        if b == 0:
            kr = blk.rotation.apply(kr_src[0], ctx)
            vr = blk.rotation.apply(vr_src[0], ctx)
        blk.cache.append_rotated(kr, vr)
        blk.host  # the host half (projection weights on the device, RoPE tables) before timing
        blocks.append(blk)
    del kr_src, vr_src
    x = torch.from_numpy(wl_rng.standard_normal((n_total, model.hidden_size)).astype(np.float32)
                         * 0.02).to(ctx.torch_device)
    ys = [None] * n_total

    def step(i):
        blk = blocks[i % a.caches]
        ys[i], _ = blk.forward(x[i], stats=False)

    for i in range(a.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.warmup, n_total):
        step(i)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / a.steps
    # the last step of its block: wire taps = the oracle's seam on the GPU's own
    # projections; out = the online softmax over the block's device rows; y to the
    # fp32 bound of the output GEMM
    last = n_total - 1
    blk = blocks[last % a.caches]
    taps = {k: t.cpu().numpy() for k, t in blk.taps.items()}
    pos = blk.cache.length - 1
    p = blk.host.project_qkv(x[last]).cpu().numpy()
    sc = model.rope_scaling
    cos, sin = oh.rope_tables(D, model.max_position, model.rope_theta,
                              scaling=oh.RopeScaling(sc.factor, sc.low_freq_factor, sc.high_freq_factor,
                                                     sc.original_max_position))
    (wq, wk, wv), _ = oh.seam(p, N_Q, N_KV, D, [pos], cos, sin)
    bad = int(not (np.array_equal(taps["wire.q"], wq) and np.array_equal(taps["wire.k"], wk)
                   and np.array_equal(taps["wire.v"], wv)))
    sg = signs_from_seed(D, 0, 1)
    qr = rotate(wq[0], sg)
    fmt = Format()
    want = np.concatenate([native.attend_online(qr[4 * h:4 * h + 4], blk.cache.view(h), fmt)[0]
                           for h in range(N_KV)])
    bad += int(not np.array_equal(taps["out"].reshape(-1), want.reshape(-1)))
    wo = blk.weights.o.cpu().numpy().view(np.float16).astype(np.float64)
    a16 = oh.to_fp16(taps["out"].reshape(1, -1) / 65536.0).astype(np.float64)
    exact = a16 @ wo.T
    tol = 2.0 * wo.shape[1] * 2.0 ** -24 * (np.abs(a16) @ np.abs(wo).T)
    bad += int(not np.all(np.abs(ys[last].cpu().numpy().astype(np.float64) - exact) <= tol))
    weights_mb = sum(b.weights.qkv.numel() * 2 + b.weights.o.numel() * 2 for b in blocks) / 2 ** 20
    cache_mb = sum(b.cache.layout()["device_total_bytes"] for b in blocks) / 2 ** 20
    res = {
        "metric": "attention block decode step (hidden in -> hidden out) at ctx 32k, 1 GPU",
        "value": round(wall * 1e6, 2), "unit": "us/token", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "higher_is_better": False, "dtype": "fp16 GEMMs, int64 seam",
        "data": "synthetic (seeded N(0,1) fp16 weights / sqrt(hidden); hidden states N(0,1) x 0.02; "
                "cache rows from the C2 generator)",
        "config": {"workload": "Llama-3.2-1B-shape attention block, batch 1, ctx 32768, 4b K / 2b V, "
                               "AttentionBlock.forward per token (projections, RoPE, cast, rotate, "
                               "append, attend, W_o')",
                   "rotating_blocks": a.caches, "rotating_mb": round(weights_mb + cache_mb, 1)},
        "check_failures": bad,
    }
    print(json.dumps(res))
    return 0 if bad == 0 else 1


def main() -> int:
    a = _args()
    if a.copy_calibration:
        copy_calibration()
        return 0
    if a.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {a.gpus}); run with --gpus 1", file=sys.stderr)
        return 2
    if a.config == "c1":
        return bench_c1(a)
    if a.config == "prefill":
        return bench_prefill(a)
    if a.config == "block":
        return bench_block(a)
    if a.config == "probe":
        return bench_probe(a)
    if a.config == "short":
        return bench_short(a)
    if a.config == "append":
        return bench_append(a)
    if a.config == "formats":
        return bench_formats(a)
    if a.config != "c2":
        return bench_scale(a)
    import torch

    from insitu_amd import ModelConfig, QuantConfig
    from insitu_amd.attention import CompressedAttention
    from insitu_amd.cache import CompressedCache
    from insitu_amd.rotate import Rotation
    from insitu_amd.runtime import default_context
    from insitu_amd.workload import Workload

    ctx = default_context(0)
    quant = QuantConfig(key_bits=4, value_bits=2)
    rot = Rotation.for_quant(quant, D)
    # Every timed step is the configuration's one decode step: the cache holds
    # ctx - 1 rows, the step appends row ctx - 1 and attends over all ctx. Steps
    # cycle through n_caches caches (--caches, at least as many as any pass has
    # steps) in one rotation that runs on across the warmup and every pass: step i
    # of the run uses cache i % n_caches, so between two uses of a cache the other
    # n_caches - 1 are read (more than twice the 256 MB Infinity Cache). Before a
    # pass every cache is rewound to ctx - 1 rows (a length reset, outside the timed
    # region). The roofline pass times TIMED_LAUNCHES attends with HIP events.
    n_ev = max(TIMED_LAUNCHES, a.steps)
    n_caches = max(a.caches, a.steps, a.warmup, n_ev, 1)
    n_tp = a.steps if a.mode == "online" else 0        # the two-pass line's steps
    n_steps_total = a.warmup + a.steps + n_ev + n_tp

    # Prefill data: ctx-1 tokens of seeded wire k/v, rotated and appended on the GPU.
    wl = Workload(seed=0)
    _, k, v = wl.steps(a.ctx - 1)
    kr = rot.apply(k[0], ctx)
    vr = rot.apply(v[0], ctx)
    qs, ks, vs = wl.steps(n_steps_total)      # the decode tokens
    del k, v
    caches = []
    for _ in range(n_caches):
        c = CompressedCache(N_KV, D, a.ctx, quant, batch=1, n_q_heads=N_Q, chunk_tokens=a.chunk_tokens, ctx=ctx)
        c.append_rotated(kr, vr)
        if a.kernel != "auto":
            c.pin_kernel(a.kernel)
        caches.append(c)
    qs_d = ctx.to_device(qs[0], torch.int32)
    ks_d = ctx.to_device(ks[0], torch.int32)
    vs_d = ctx.to_device(vs[0], torch.int32)
    torch.cuda.synchronize()
    total_mb = sum(c.layout()["device_total_bytes"] for c in caches) / 2 ** 20

    outs = [torch.empty((1, N_Q, D), dtype=torch.int32, device=ctx.torch_device)
            for _ in range(n_steps_total)]
    lib = ctx.lib
    from insitu_amd import _lib
    from insitu_amd.runtime import ptr
    import ctypes
    mode = _lib.MODES[a.mode]
    step_bytes = float(N_KV * ROW * a.ctx)      # the rows one attend scans

    def step(i, md=None):
        # One decode step from the wire, CMD_STEP (kernel.py:271-345): rotate q/k/v,
        # append the k/v row, attend -- one launch in online mode. Step i of the run
        # takes cache i % n_caches.
        _lib.check(lib.insitu_step(caches[i % n_caches].handle, ptr(qs_d[i]), ptr(ks_d[i]), ptr(vs_d[i]),
                                   ptr(outs[i]), mode if md is None else md, None))

    def rewind():
        for c in caches:
            c.set_length(a.ctx - 1)
        torch.cuda.synchronize()

    def timed_pass(i0, n, timing, md=None):
        rewind()
        _lib.check(lib.insitu_ctx_timing(ctx.handle, 1 if timing else 0))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for j in range(n):
            step(i0 + j, md)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = (ctypes.c_double * n)()
        n_att = ctypes.c_int64()
        _lib.check(lib.insitu_ctx_timing_read_each(ctx.handle, ms, n, ctypes.byref(n_att)))
        _lib.check(lib.insitu_ctx_timing(ctx.handle, 0))
        if n_att.value != (n if timing else 0):
            raise RuntimeError(f"timed {n_att.value} attends for {n} steps")
        return wall, np.array(ms[:n_att.value]) * 1e3

    for i in range(a.warmup):
        step(i)
    torch.cuda.synchronize()
    # value: K steps with nothing attached; roofline: the attend kernel's own time,
    # from HIP events attached to its dispatches on the stream it runs on
    # (insitu_ctx_timing), over a pass of TIMED_LAUNCHES steps (the events themselves
    # cost the step a few microseconds, so that pass is not `value`)
    wall, _ = timed_pass(a.warmup, a.steps, False)
    wall_ev, us_each = timed_pass(a.warmup + a.steps, n_ev, True)
    us_med = float(np.median(us_each))
    us_mean = float(us_each.mean())
    kernel_gbs = step_bytes / (us_med * 1e-6) / 1e9
    whole_gbs = step_bytes * a.steps / wall / 1e9

    # Correctness of the timed work: the roofline pass's last step against the oracle
    # (and the CPU baseline).
    last = a.warmup + a.steps + n_ev - 1
    out_last = outs[last].cpu().numpy()[0].astype(np.int64)
    cache_last = caches[last % n_caches]
    if cache_last.length != a.ctx:
        raise RuntimeError(f"the last step's cache holds {cache_last.length} rows, not {a.ctx}")
    from oracle import native
    from oracle.quantize import Format
    q_rot_last = rotate_q(qs[0, last])
    want = np.concatenate([native.attend_online(q_rot_last[4 * h:4 * h + 4], cache_last.view(h), Format())[0]
                           for h in range(N_KV)]) if a.mode != "two_pass" else None
    if want is not None and not np.array_equal(want, out_last):
        raise AssertionError("the last timed step disagrees with the oracle")
    # (before the two-pass line below, whose pass rewinds every cache to ctx - 1 rows)
    cpu = None
    if not a.no_cpu_baseline:
        cpu = cpu_baseline(cache_last, q_rot_last, out_last, (qs[0, last], ks[0, last], vs[0, last]))
    # The adapter's default softmax is two-pass (three launches a step): its line, K steps
    # on the same rotation, checked against the oracle's attend_two_pass.
    two_pass = None
    if n_tp:
        i0 = last + 1
        wall_tp, _ = timed_pass(i0, n_tp, False, _lib.MODES["two_pass"])
        i_tp = i0 + n_tp - 1
        q_tp = rotate_q(qs[0, i_tp])
        c_tp = caches[i_tp % n_caches]
        want_tp = np.concatenate([native.attend_two_pass(q_tp[4 * h:4 * h + 4], c_tp.view(h), Format())[0]
                                  for h in range(N_KV)])
        if not np.array_equal(want_tp, outs[i_tp].cpu().numpy()[0].astype(np.int64)):
            raise AssertionError("the two-pass line's last step disagrees with the oracle")
        two_pass = {"mode": "two_pass", "steps": n_tp,
                    "kernels": STEP_KERNEL["two_pass"],
                    "us_per_decode_step": round(wall_tp / n_tp * 1e6, 2),
                    "GB/s": round(step_bytes * n_tp / wall_tp / 1e9, 3),
                    "checked": "the last step equal to oracle/c attend_two_pass"}
    kernel = STEP_KERNEL.get(a.mode, a.mode)
    if a.kernel == "chunked" and a.mode in ("online", "split"):
        kernel = CHUNKED_STEP_KERNEL
    traffic, traffic_src = measured_traffic(kernel, a.ctx)
    cache_mb = total_mb / n_caches

    res = {
        "metric": "compressed-KV scan GB/s (% HBM peak) + us/decode-step at ctx 32k, 1 GPU",
        "value": round(whole_gbs, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(wall / a.steps * 1e3, 4),
        "us_per_decode_step": round(wall / a.steps * 1e6, 2),
        "us_per_decode_step_timing_pass": round(wall_ev / a.steps * 1e6, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int64",
        "data": "synthetic (seeded N(0,1) q/k/v with 4 outlier channels x8 per head, Q8.16)",
        "config": {"workload": "C2: Llama-3.2-1B-shape single layer, batch 1, ctx 32768, "
                               "4b K / 2b V, decode step = insitu_step: rotate + append + attend",
                   "mode": a.mode, "kernel": a.kernel, "chunk_tokens": a.chunk_tokens or 1024, "ctx": a.ctx,
                   "rotating_caches": n_caches, "rotating_mb": round(total_mb, 1),
                   "caches_per_timed_pass": min(a.steps, n_caches),
                   "reuse_distance_mb": round(cache_mb * (n_caches - 1), 1),
                   "kv_heads": N_KV, "q_heads": N_Q, "head_dim": D, "row_bytes": ROW},
        "roofline": {"bound": "hbm", "achieved": round(kernel_gbs, 3), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kernel_gbs / HBM_PEAK_GBS, 5),
                     "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": kernel,
                     "algorithmic_bytes_per_launch": step_bytes,
                     "attend_us_median": round(us_med, 3),
                     "attend_us_mean": round(us_mean, 3),
                     "attend_us_min": round(float(us_each.min()), 3),
                     "attend_us_max": round(float(us_each.max()), 3),
                     "event_timed_launches": int(us_each.size),
                     "cycles_per_row_gpu_wide_2p4ghz": round(
                         us_med * 1e-6 * 2.4e9 / (step_bytes / ROW), 4),
                     "cycles_per_row_per_cu_2p4ghz": round(
                         us_med * 1e-6 * 2.4e9 * N_CU / (step_bytes / ROW), 2)},
        "checked": "the last timed step equal to oracle/c attend_online" if want is not None else None,
        "two_pass_line": two_pass,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())
