"""Phase breakdown of the decode step kernel (attend_step.hip), from its phase stamps.

    python -m insitu_amd.build --stamps       # once, on the build host
    python -m insitu_amd.phases [short] [c2] [c2flat]

The stamped library (libinsitu_hip_stamps.so) is the product library with
INSITU_STEP_STAMPS defined for attend_step.hip: lane 0 of every wave writes
s_memrealtime (100 MHz) at each phase boundary into a device array, which this
module reads back after each step. Nothing else of the kernel changes. Each
case rewinds a cache to ctx - 1 rows and runs insitu_step on it (q/k/v of the
C2 workload), once per repetition, rotating over several caches; times are in
microseconds from the earliest wave start of the launch.

For every phase it prints the median over repetitions of the per-workgroup time
(the last wave of the workgroup to pass the point), then the median, minimum and
maximum of that over the workgroups, and the same for wave 0 of the workgroup
that replays chain 0 (the sequence's last chunk).
"""

from __future__ import annotations

import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
NWAVES, NSTAMPS, MAXBLK = 16, 32, 8192

# stamp index -> the point of the kernel it marks
PHASES = [
    (0, "start"),
    (1, "P0 loads, query rotation, new row"),
    (2, "barrier B1"),
    (3, "P1 scores and wave maxima"),
    (4, "barrier B2"),
    (5, "P2 look-back (barrier B3)"),
    (17, "P3 chunk 0: list test"),
    (18, "P3 chunk 0: barrier L1"),
    (19, "P3 chunk 0: list compacted"),
    (21, "P3 list: barrier L2"),
    (20, "P3 list: pass (events, p, terms)"),
    (16, "P3 chunk 0 folded from its list"),
    (11, "P3 event scan (barrier B4)"),
    (13, "P3 candidates, terms (barrier B5)"),
    (6, "P3 run sums, candidate list (B6)"),
    (7, "P4 walk (barrier B7)"),
    (12, "P5 runs and header published (other chunks)"),
    (8, "P5 own fold or publish"),
    (14, "P6 headers read"),
    (15, "P6 runs staged"),
    (23, "P6 block sums scanned"),
    (30, "P6 runs walked (before own runs)"),
    (9, "P6 replay walked"),
    (31, "P6 output row stored"),
    (10, "end (finalize)"),
]


def _load():
    import torch  # noqa: F401  (the HIP runtime through torch first)
    from insitu_amd import _lib
    path = os.path.join(HERE, "libinsitu_hip_stamps.so")
    lib = _lib.load(path)
    if not hasattr(lib, "insitu_step_stamps_read"):
        raise RuntimeError(f"{path} has no phase stamps; build it with python -m insitu_amd.build --stamps")
    lib.insitu_step_stamps_read.argtypes = [ctypes.c_void_p, ctypes.c_long]
    return lib


def run(ctx_len: int, n_caches: int, reps: int, flat: bool = False) -> dict:
    import torch
    from insitu_amd import QuantConfig, _lib
    from insitu_amd.cache import CompressedCache
    from insitu_amd.rotate import Rotation
    from insitu_amd.runtime import default_context, ptr
    from insitu_amd.workload import Workload

    lib = _load()
    ctx = default_context(0)
    quant = QuantConfig(key_bits=4, value_bits=2)
    rot = Rotation.for_quant(quant, 64)
    wl = Workload(seed=0)
    _, k, v = wl.steps(ctx_len - 1)
    kr, vr = rot.apply(k[0], ctx), rot.apply(v[0], ctx)
    qs, ks, vs = wl.steps(reps + 4)
    if flat:
        qs = qs >> 9
    caches = []
    for _ in range(n_caches):
        c = CompressedCache(8, 64, max(ctx_len, 256), quant, n_q_heads=32, ctx=ctx)
        c.append_rotated(kr, vr)
        c.pin_kernel("step")
        caches.append(c)
    q = ctx.to_device(qs[0], torch.int32)
    kw = ctx.to_device(ks[0], torch.int32)
    vw = ctx.to_device(vs[0], torch.int32)
    out = torch.empty((32, 64), dtype=torch.int32, device=ctx.torch_device)
    nch = (ctx_len + 1023) // 1024
    nblk = nch * 8
    buf = np.zeros(MAXBLK * NWAVES * NSTAMPS, dtype=np.uint64)
    runs, counts, rcounts = [], [], []
    for i in range(reps + 4):
        c = caches[i % n_caches]
        c.set_length(ctx_len - 1)
        torch.cuda.synchronize()
        lib.insitu_step_stamps_clear()
        torch.cuda.synchronize()
        _lib.check(lib.insitu_step(c.handle, ptr(q[i]), ptr(kw[i]), ptr(vw[i]), ptr(out), 0, None))
        torch.cuda.synchronize()
        lib.insitu_step_stamps_read(buf.ctypes.data, buf.size)
        if i < 4:
            continue                                   # warmup
        st = buf[:nblk * NWAVES * NSTAMPS].reshape(nblk, NWAVES, NSTAMPS).astype(np.int64)
        counts.append(st[:, :4, 24:27].copy())          # head waves: list entries, tokens of weight, events
        rcounts.append(st[:, :4, 27:29].copy())         # replay: runs walked, certified (1) or not (2)
        st[:, :, 24:29] = 0
        t0 = st[:, :, 0][st[:, :, 0] > 0].min()
        runs.append(np.where(st > 0, (st - t0) * 0.01, np.nan))
    R = np.stack(runs)                                  # (reps, block, wave, stamp), us
    with np.errstate(all="ignore"), __import__("warnings").catch_warnings():
        __import__("warnings").simplefilter("ignore")
        per_blk = np.nanmedian(np.nanmax(R, axis=2), axis=0)     # (block, stamp)
        rep_blk = (nch - 1) * 8                                  # chain 0's last chunk
        w0 = np.nanmedian(R[:, rep_blk, 0], axis=0)               # (stamp,)
    C = np.stack(counts[4:]) if len(counts) > 4 else None          # (reps, block, head, 3)
    RC = np.stack(rcounts[4:])[:, (nch - 1) * 8:] if len(rcounts) > 4 else None    # the replaying workgroups
    return {"ctx": ctx_len, "flat": flat, "reps": reps, "blocks": nblk, "per_blk": per_blk, "replayer_w0": w0,
            "counts": C, "rcounts": RC}


def table(res: dict) -> str:
    def f(x):
        return "-" if np.isnan(x) else f"{x:.2f}"
    lines = [f"ctx {res['ctx']}{' (flat softmax)' if res['flat'] else ''}: {res['blocks']} workgroups, "
             f"median of {res['reps']} steps, us from the launch's first wave",
             "",
             "| stamp | point | workgroups: median | min | max | replaying workgroup, wave 0 | chunk 0 (median over KV heads) |",
             "|---|---|---|---|---|---|---|"]
    for k, name in PHASES:
        col = res["per_blk"][:, k]
        if np.all(np.isnan(col)) and np.isnan(res["replayer_w0"][k]):
            continue
        with np.errstate(all="ignore"), __import__("warnings").catch_warnings():
            __import__("warnings").simplefilter("ignore")
            c0 = np.nanmedian(col[:8]) if res["blocks"] > 8 else np.nan
            lines.append(f"| {k} | {name} | {f(np.nanmedian(col))} | {f(np.nanmin(col))} | "
                         f"{f(np.nanmax(col))} | {f(res['replayer_w0'][k])} | {f(c0)} |")
    C = res.get("counts")
    if C is not None and C.any():
        c0, rest = C[:, :8], C[:, 8:]
        lines += ["", "chunk list per head (median over steps; chunk 0 / other chunks): "
                  f"entries {np.median(c0[..., 0]):.0f} (max {c0[..., 0].max()}) / {np.median(rest[..., 0]) if rest.size else 0:.1f} "
                  f"(max {rest[..., 0].max() if rest.size else 0}), tokens of weight {np.median(c0[..., 1]):.0f} "
                  f"(max {c0[..., 1].max()}) / {np.median(rest[..., 1]) if rest.size else 0:.1f}, "
                  f"events {np.median(c0[..., 2]):.0f} (max {c0[..., 2].max()})"]
    RC = res.get("rcounts")
    if RC is not None and (RC[..., 0] > 0).any():
        walked = RC[..., 0][RC[..., 0] > 0]
        lines += ["", f"replay per head: runs of the other chunks walked, median {np.median(walked):.0f} "
                  f"(max {walked.max()}); certified at once in {(RC[..., 1] == 1).sum()} of {(RC[..., 1] > 0).sum()}"]
    pub = res["per_blk"][:, 12]
    if res["blocks"] > 8 and not np.all(np.isnan(pub)):
        order = np.argsort(np.nan_to_num(pub, nan=-1.0))[::-1][:6]
        lines += ["", "last chunks to publish (chunk, KV head, us): " +
                  ", ".join(f"({b // 8}, {b % 8}, {pub[b]:.2f})" for b in order)]
    return "\n".join(lines)


def main(argv) -> int:
    cases = argv or ["short", "c2"]
    for c in cases:
        if c == "short":
            res = run(100, 4, 20)
        elif c == "c2":
            res = run(32768, 24, 20)
        elif c == "c2flat":
            res = run(32768, 24, 10, flat=True)
        else:
            raise SystemExit(f"unknown case {c}")
        print(table(res))
        print()
        sys.stdout.flush()
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
