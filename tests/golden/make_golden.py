#!/usr/bin/env python3
"""Write the golden fixtures of tests/golden/ from the RustFox reference.

The reference is compiled from its own sources by oracle/Makefile into
oracle/_ref/libfoxref.so (baseline x86-64, so no FMA contraction) and called
through ctypes; nothing of it is copied here.  Each fixture holds seeded
inputs and the reference's outputs:

  gemv_<type>.npz     weights, activations x, fox_gemv outputs (and for the
                      TQ types the int8 activations and scale of
                      fox_quantize_activations_i8)
  quantize.npz        fox_quantize_activations_i8 on edge vectors
  decode_tiny.npz     a 2-layer tiny-512 synthetic model (its GGUF sha256),
                      prompt logits of fox_eval and 16 greedy ids

Run:  make -C oracle ref && python tests/golden/make_golden.py
"""
import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from oracle_libs import Ref  # noqa: E402
from rustfox_amd import synth  # noqa: E402

TYPES = {"tq1_0": 34, "tq2_0": 35, "q4_k": 12, "q6_k": 14, "f16": 1}


def weights(rng, gtype, N, K):
    if gtype in (34, 35):
        bb = 54 if gtype == 34 else 66
        w = rng.integers(0, 256, size=(N * K // 256, bb), dtype=np.uint8)
        w[:, bb - 2:] = rng.uniform(0.01, 0.05, size=w.shape[0]).astype(np.float16).view(
            np.uint8).reshape(-1, 2)
        return w.reshape(-1)
    if gtype == 12:
        return synth.q4k_quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.02).reshape(-1)
    if gtype == 14:
        return synth.q6k_quantize(rng.standard_normal((N, K)).astype(np.float32) * 0.02).reshape(-1)
    return (rng.standard_normal((N, K)) * 0.02).astype(np.float16).view(np.uint8).reshape(-1)


def main():
    ref = Ref()
    shapes = {"tq1_0": (37, 512), "tq2_0": (37, 512), "q4_k": (33, 768), "q6_k": (29, 512),
              "f16": (50, 288)}
    for name, (N, K) in shapes.items():
        gtype = TYPES[name]
        rng = np.random.default_rng([0x601D, gtype])
        w = weights(rng, gtype, N, K)
        x = rng.standard_normal((3, K)).astype(np.float32)
        out = np.stack([ref.gemv(gtype, x[t], w, N, K, n_threads=1) for t in range(3)])
        extra = {}
        if gtype in (34, 35):
            qs = [ref.quantize(x[t]) for t in range(3)]
            extra = {"q": np.stack([q for q, _ in qs]),
                     "scale": np.array([s for _, s in qs], np.float32)}
        np.savez_compressed(os.path.join(HERE, f"gemv_{name}.npz"), w=w, x=x, out=out,
                            rows=N, cols=K, gtype=gtype, **extra)
        print(f"gemv_{name}.npz: {N}x{K}")

    vecs = [np.zeros(512, np.float32), (np.arange(512, dtype=np.float32) - 200.0),
            np.random.default_rng(1).standard_normal(4096).astype(np.float32) * 37.5]
    qd = {}
    for i, v in enumerate(vecs):
        q, s = ref.quantize(v)
        qd[f"x{i}"], qd[f"q{i}"], qd[f"s{i}"] = v, q, np.float32(s)
    np.savez_compressed(os.path.join(HERE, "quantize.npz"), **qd)
    print("quantize.npz")

    spec = synth.spec("tiny-512", n_layer=2, n_vocab=2000)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "tiny.gguf")
        synth.write_gguf(path, spec)
        sha = hashlib.sha256(open(path, "rb").read()).hexdigest()
        m = ref.open_model(path)
        ctx = m.context(64, n_batch=32, n_threads=1)
        prompt = synth.prompt_ids(16, spec.n_vocab)
        logits = ctx.eval(prompt)
        ids, lg = [], logits
        for _ in range(16):
            ids.append(int(np.argmax(lg)))
            lg = ctx.eval(np.array([ids[-1]], np.uint32))
        ctx.close()
        m.close()
    np.savez_compressed(os.path.join(HERE, "decode_tiny.npz"), sha256=sha, prompt=prompt,
                        logits=logits, ids=np.array(ids, np.uint32))
    print("decode_tiny.npz:", sha[:16], ids[:6])


if __name__ == "__main__":
    main()
