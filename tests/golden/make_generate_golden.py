"""Writes tests/golden/generate_<name>.json: the reference's greedy generation
for a deterministic random checkpoint (tests/golden/make_checkpoint.py).

Two reference runs, both built from the StrataKV sources by oracle/Makefile:
* oracle/_ref/libstratakv_ref.so :: ref_generate_trace -- the reference's CPU
  generation path (load_safetensors, TransformerBlock::forward, RMSNorm,
  Linear) driven step by step, recording the greedy token and the top-8
  logits of every step;
* oracle/_ref/stratakv_cli -- the reference's own command-line program
  (1024-block pool, block size 16, EOS 2), whose printed tokens must equal the
  trace's up to its EOS stop.
The fixture holds the checkpoint spec and SHA-256, the prompt
(numpy default_rng(42).integers(0, vocab, 16)), the generated tokens, and the
per-step top-8 ids and logits.  This container only (the reference sources and
their build are not on the GPU box); a TinyLlama run takes ~25 min of CPU.

Usage: python tests/golden/make_generate_golden.py {mini|tinyllama} N_NEW [CKPT_DIR]
"""
from __future__ import annotations

import ctypes
import json
import os
import subprocess
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, HERE)
import make_checkpoint  # noqa: E402

TOP_K = 8
EOS = 2  # the reference CLI's EOS id (src/cli.cpp:279)


def main() -> None:
    name, n_new = sys.argv[1], int(sys.argv[2])
    ckpt_dir = sys.argv[3] if len(sys.argv) > 3 else "/tmp/skv_ckpt"
    g = make_checkpoint.GEOMETRIES[name]
    path, sha = make_checkpoint.ensure(name, ckpt_dir)
    prompt = [int(x) for x in np.random.default_rng(42).integers(0, g["vocab"], 16)]

    cli = subprocess.Popen([os.path.join(ROOT, "oracle", "_ref", "stratakv_cli"), path, str(n_new),
                            *map(str, prompt)], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "_ref", "libstratakv_ref.so"))
    toks = np.array(prompt + [-1] * n_new, np.int32)
    steps = n_new + 1
    am = np.zeros(steps, np.int32)
    ids = np.zeros(steps * TOP_K, np.int32)
    vals = np.zeros(steps * TOP_K, np.float32)
    err = ctypes.create_string_buffer(512)
    vp = ctypes.c_void_p
    t0 = time.time()
    rc = lib.ref_generate_trace(path.encode(), g["layers"], g["heads"], g["kv_heads"], toks.ctypes.data_as(vp),
                                len(toks), len(prompt), TOP_K, am.ctypes.data_as(vp), ids.ctypes.data_as(vp),
                                vals.ctypes.data_as(vp), err, 512)
    trace_s = time.time() - t0
    if rc != 0:
        sys.exit(f"ref_generate_trace failed: {err.value.decode()}")
    out, cli_err = cli.communicate()
    if cli.returncode != 0:
        sys.exit(f"stratakv_cli failed: {cli_err}")
    cli_tokens = [int(x) for x in out.split()]
    generated = [int(x) for x in toks[len(prompt):]]
    # The CLI stops after an EOS token; the trace does not.
    expect = list(prompt)
    for tok in generated:
        expect.append(tok)
        if tok == EOS:
            break
    if cli_tokens != expect:
        sys.exit(f"reference CLI and trace disagree:\n{cli_tokens}\n{expect}")
    fixture = {
        "checkpoint": {"geometry": name, **g, "sha256": sha, "writer": "tests/golden/make_checkpoint.py"},
        "prompt": prompt,
        "generated": generated,
        "cli_tokens": cli_tokens,
        "eos": EOS,
        "top_k": TOP_K,
        "top_ids": ids.reshape(steps, TOP_K).tolist(),
        "top_vals": [[float(v) for v in row] for row in vals.reshape(steps, TOP_K)],
        "reference_cpu_seconds": round(trace_s, 1),
        "cli_timing": [l for l in cli_err.splitlines() if l.startswith("[")],
    }
    dst = os.path.join(HERE, f"generate_{name}.json")
    with open(dst, "w") as f:
        json.dump(fixture, f, indent=None, separators=(",", ":"))
        f.write("\n")
    print(f"wrote {dst}: {len(generated)} tokens, trace {trace_s:.1f} s")


if __name__ == "__main__":
    main()
