"""Write the golden vectors the reference's own fixtures do not hold.

Run once, in a build container where the reference checkout is readable (it is
never read at test time and never travels to a GPU box):

    python tests/golden/make_reference_vectors.py /root/reference

The reference ships `tb/vectors/` for one configuration only (Llama-3.2-1B shape,
4-bit keys, 2-bit values, ctx 64 + 1). Nothing there pins:
  - `Codebook.gaussian(bits)` for widths other than 2 and 4 (ops/codebook.py:67-120),
    in particular the 3-bit codebook config 4 uses;
  - a d = 128 block (Llama-3-8B's attention shape) with 3-bit keys and values;
  - a config-0-shaped step (ctx 512 + 1);
  - decode steps from an empty cache.
This script imports the reference's numpy model and records those, with the
reference's own generator order (hw/vectors.py:821-841 `build`, :199-304
`collect`), into small fixtures beside it:

    codebooks_gaussian.json        Codebook.gaussian(b) integers, b = 1 .. 8
    d128_3b3b_ctx64.npz            one collect() step, Llama-3-8B attention shape
    d64_4b2b_ctx512.npz            one collect() step at config 0's context
    d64_4b2b_steps_from_empty.npz  the first 40 decode steps of an empty cache

Each .npz holds integers only and loads with numpy.load(allow_pickle=False).
"""

from __future__ import annotations

import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _import_reference(root: str):
    """The reference is a package named `kernel` (its tests do `from kernel import ...`)."""
    tmp = tempfile.mkdtemp(prefix="insitu_ref_")
    os.symlink(os.path.abspath(root), os.path.join(tmp, "kernel"))
    sys.path.insert(0, tmp)
    import kernel.config as config  # noqa: F401
    from kernel.hw import vectors
    from kernel.kernel import AttentionKernel
    from kernel.ops.codebook import Codebook
    return config, vectors, AttentionKernel, Codebook


def _step_arrays(vs) -> dict:
    """The integer stages of one collect() step (hw/vectors.py:144-196 VectorSet)."""
    out = {
        "context": np.array(vs.context, dtype=np.int64),
        "wire_q": np.asarray(vs.wire["q"], dtype=np.int64),
        "wire_k": np.asarray(vs.wire["k"], dtype=np.int64),
        "wire_v": np.asarray(vs.wire["v"], dtype=np.int64),
        "rot_q": np.asarray(vs.rotated["q"], dtype=np.int64),
        "rot_k": np.asarray(vs.rotated["k"], dtype=np.int64),
        "rot_v": np.asarray(vs.rotated["v"], dtype=np.int64),
        "row": np.asarray(vs.rows, dtype=np.uint8),              # the appended row, (n_kv, row_bytes)
        "cache": np.asarray(vs.cache, dtype=np.uint8),           # (ctx + 1, n_kv, row_bytes)
        "scores": np.asarray(vs.scores, dtype=np.int64),         # (n_q, ctx + 1)
        "out_online": np.asarray(vs.out_online, dtype=np.int64),  # (1, n_q * d), merge_heads order
        "out_two_pass": np.asarray(vs.out_two_pass, dtype=np.int64),
        "final_acc": np.asarray(vs.final["acc"], dtype=np.int64),
        "final_l": np.asarray(vs.final["l"], dtype=np.int64),
    }
    q = vs.quantizer
    out["key_centroids"] = np.asarray(q.key.codebook.centroids, dtype=np.int64)
    out["key_bounds"] = np.asarray(q.key.codebook.boundaries, dtype=np.int64)
    out["value_centroids"] = np.asarray(q.value.codebook.centroids, dtype=np.int64)
    out["value_bounds"] = np.asarray(q.value.codebook.boundaries, dtype=np.int64)
    return out


def _build(config, vectors, AttentionKernel, *, hidden, heads, kv_heads, d, ctx, kb, vb, seed=0):
    """hw/vectors.py:821-841 `build`, at a given attention shape."""
    m = config.ModelConfig(hidden_size=hidden, num_heads=heads, num_kv_heads=kv_heads, head_dim=d,
                           max_position=max(4096, ctx * 2 + 2))
    cfg = config.KernelConfig(model=m, quant=config.QuantConfig(key_bits=kb, value_bits=vb, seed=seed))
    k = AttentionKernel(cfg, capacity=ctx + 1)
    rng = np.random.default_rng(seed)
    if ctx:
        k.forward(rng.standard_normal((ctx, m.hidden_size)).astype(np.float32) * 0.02)
    step = rng.standard_normal((1, m.hidden_size)).astype(np.float32) * 0.02
    return vectors.collect(k, step)


def main(argv=None) -> int:
    root = (argv or sys.argv[1:] or ["/root/reference"])[0]
    config, vectors, AttentionKernel, Codebook = _import_reference(root)

    books = {}
    for b in range(1, 9):
        cb = Codebook.gaussian(b)
        books[str(b)] = {"centroids": [int(x) for x in cb.centroids],
                         "boundaries": [int(x) for x in cb.boundaries], "frac": int(cb.frac)}
    with open(os.path.join(HERE, "codebooks_gaussian.json"), "w") as f:
        json.dump({"source": "ops/codebook.py:67-120 Codebook.gaussian(bits), frac 15, symmetric",
                   "codebooks": books}, f, indent=1)
    print("codebooks_gaussian.json: widths 1 .. 8")

    # Llama-3-8B attention shape (32 query heads, 8 KV heads, d = 128, hidden 4096), 3b/3b
    vs = _build(config, vectors, AttentionKernel, hidden=4096, heads=32, kv_heads=8, d=128, ctx=64, kb=3, vb=3)
    np.savez_compressed(os.path.join(HERE, "d128_3b3b_ctx64.npz"), **_step_arrays(vs))
    print("d128_3b3b_ctx64.npz: ctx 64 + 1, row", vs.rows.shape)

    # config 0's context: Llama-3.2-1B shape, 4b/2b, ctx 512 + 1
    vs = _build(config, vectors, AttentionKernel, hidden=2048, heads=32, kv_heads=8, d=64, ctx=512, kb=4, vb=2)
    np.savez_compressed(os.path.join(HERE, "d64_4b2b_ctx512.npz"), **_step_arrays(vs))
    print("d64_4b2b_ctx512.npz: ctx 512 + 1")

    # decode steps from an empty cache: one collect() per token, as many steps
    m = config.ModelConfig(hidden_size=2048, num_heads=32, num_kv_heads=8, head_dim=64, max_position=4096)
    cfg = config.KernelConfig(model=m, quant=config.QuantConfig(key_bits=4, value_bits=2, seed=0))
    n = 40
    k = AttentionKernel(cfg, capacity=n)
    rng = np.random.default_rng(1)
    xs = rng.standard_normal((n, m.hidden_size)).astype(np.float32) * 0.02
    wq, wk, wv, outs, rows = [], [], [], [], []
    for t in range(n):
        vs = vectors.collect(k, xs[t:t + 1])
        wq.append(vs.wire["q"][0])
        wk.append(vs.wire["k"][0])
        wv.append(vs.wire["v"][0])
        outs.append(vs.out_online[0])
        rows.append(vs.rows)
    np.savez_compressed(os.path.join(HERE, "d64_4b2b_steps_from_empty.npz"),
                        wire_q=np.asarray(wq, dtype=np.int64), wire_k=np.asarray(wk, dtype=np.int64),
                        wire_v=np.asarray(wv, dtype=np.int64), out_online=np.asarray(outs, dtype=np.int64),
                        rows=np.asarray(rows, dtype=np.uint8))
    print(f"d64_4b2b_steps_from_empty.npz: {n} steps")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
