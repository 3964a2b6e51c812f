"""Deterministic random Llama checkpoints in safetensors format (test data).

A checkpoint is fully defined by its geometry and seed, so the files are never
committed: the tests regenerate them (here and on the GPU box) and check the
SHA-256 recorded beside the golden token streams.

Layout (the Hugging Face Llama schema the reference's loader and Generator
read, src/generation/generator.cpp:387-461, src/cli.cpp:80-140):
  model.embed_tokens.weight            [vocab, hidden]
  model.layers.{i}.input_layernorm.weight          [hidden]
  model.layers.{i}.self_attn.{q,k,v,o}_proj.weight [out, in]
  model.layers.{i}.post_attention_layernorm.weight [hidden]
  model.layers.{i}.mlp.{gate,up,down}_proj.weight  [out, in]
  model.norm.weight                    [hidden]
  lm_head.weight                       [vocab, hidden]
in that order, all BF16.  Matrices are numpy PCG64(seed).standard_normal
(float32) * 0.02 drawn in that order, rounded to nearest-even bf16; norm
gammas are 1.0.  The JSON header is padded with spaces to a multiple of 8
bytes.

Usage: python tests/golden/make_checkpoint.py {tinyllama|mini|small} OUT.safetensors
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
import sys

import numpy as np

GEOMETRIES = {
    # config 1: TinyLlama-1.1B shape
    "tinyllama": dict(layers=22, hidden=2048, heads=32, kv_heads=4, ffn=5632, vocab=32000, seed=1234),
    # small model for fast CPU/GPU tests (head_dim 64, GQA group 2)
    "mini": dict(layers=2, hidden=256, heads=4, kv_heads=2, ffn=512, vocab=1000, seed=77),
    # small model whose projections take the fused one-token kernels (inputs of
    # at least 512): the decode step the Generator replays from a graph
    "small": dict(layers=3, hidden=512, heads=8, kv_heads=2, ffn=1024, vocab=2000, seed=91),
}


def tensor_list(g: dict) -> list[tuple[str, tuple[int, ...], bool]]:
    """(name, shape, is_norm) in file and draw order."""
    h, hd = g["hidden"], g["hidden"] // g["heads"]
    kv = g["kv_heads"] * hd
    out = [("model.embed_tokens.weight", (g["vocab"], h), False)]
    for i in range(g["layers"]):
        p = f"model.layers.{i}."
        out += [
            (p + "input_layernorm.weight", (h,), True),
            (p + "self_attn.q_proj.weight", (h, h), False),
            (p + "self_attn.k_proj.weight", (kv, h), False),
            (p + "self_attn.v_proj.weight", (kv, h), False),
            (p + "self_attn.o_proj.weight", (h, h), False),
            (p + "post_attention_layernorm.weight", (h,), True),
            (p + "mlp.gate_proj.weight", (g["ffn"], h), False),
            (p + "mlp.up_proj.weight", (g["ffn"], h), False),
            (p + "mlp.down_proj.weight", (h, g["ffn"]), False),
        ]
    out += [("model.norm.weight", (h,), True), ("lm_head.weight", (g["vocab"], h), False)]
    return out


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (finite inputs)."""
    b = x.astype(np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def write(name: str, path: str) -> str:
    """Write the checkpoint; returns its SHA-256 (hex)."""
    g = GEOMETRIES[name]
    entries = tensor_list(g)
    header, off = {}, 0
    for tname, shape, _ in entries:
        n = int(np.prod(shape)) * 2
        header[tname] = {"dtype": "BF16", "shape": list(shape), "data_offsets": [off, off + n]}
        off += n
    hj = json.dumps(header, separators=(",", ":")).encode()
    hj += b" " * (-len(hj) % 8)
    rng = np.random.default_rng(g["seed"])
    sha = hashlib.sha256()
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        for chunk in (struct.pack("<Q", len(hj)), hj):
            f.write(chunk)
            sha.update(chunk)
        for _, shape, is_norm in entries:
            if is_norm:
                data = np.full(shape, 0x3F80, np.uint16)   # 1.0
            else:
                data = bf16_rne(rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))
            raw = data.astype("<u2").tobytes()
            f.write(raw)
            sha.update(raw)
    os.replace(tmp, path)
    return sha.hexdigest()


def ensure(name: str, directory: str) -> tuple[str, str]:
    """Path of the `name` checkpoint under `directory`, written if missing
    (a `.sha256` file beside it caches the hash); returns (path, sha256)."""
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, f"{name}.safetensors")
    sha_path = path + ".sha256"
    if os.path.exists(path) and os.path.exists(sha_path):
        with open(sha_path) as f:
            return path, f.read().strip()
    sha = write(name, path)
    with open(sha_path, "w") as f:
        f.write(sha + "\n")
    return path, sha


if __name__ == "__main__":
    if len(sys.argv) != 3 or sys.argv[1] not in GEOMETRIES:
        sys.exit(__doc__)
    print(write(sys.argv[1], sys.argv[2]))
