"""The model boundary on the device: checkpoint decode kernels and the device
loader, the embedding lookup, greedy and sampled token choice, and the
Generator end to end against the reference's own greedy generations
(tests/golden/generate_*.json, written by tests/golden/make_generate_golden.py
from the reference CLI and the reference's CPU forward).

Tolerances:
* checkpoint decode, embedding, argmax: bit-exact / exact;
* sampler: the same token as the reference restatement (oracle/sampler.py,
  pinned against the reference's Sampler) unless the draw or top_p lies within
  1e-5 of a cumulative boundary (the kernel sums masses in double, in another
  order than the reference's float loops);
* logits: the reference computes in fp32 with an fp32 KV cache, this build
  keeps the cache in bf16 (its RNE rounding perturbs every attention read by
  up to 2^-9 relative), so logits are compared with |d| <= 2e-2 + 2e-2 |ref|,
  and greedy tokens must match the reference's wherever the reference's own
  top-2 gap exceeds twice that bound.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import stratakv_amd as skv
import oracle
from oracle import sampler as osamp

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.path.join(ROOT, "build", "bin", "tool_model")
GOLDEN = os.path.join(ROOT, "tests", "golden")
sys.path.insert(0, GOLDEN)
import make_checkpoint  # noqa: E402

LOGIT_ABS, LOGIT_REL = 2e-2, 2e-2


def tool(*args, timeout=600):
    p = subprocess.run([TOOL, *map(str, args)], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                       timeout=timeout)
    assert p.returncode == 0, p.stderr
    return json.loads(p.stdout.strip().splitlines()[-1])


# ---------------------------------------------------------------------------
# kernels through the C ABI
# ---------------------------------------------------------------------------
def test_convert_kernels_bit_exact(gpu):
    rng = np.random.default_rng(3)
    halves = np.concatenate([np.array([0, 0x8000, 1, 0x8001, 0x3FF, 0x200, 0x400, 0x7BFF, 0x7C00, 0xFC00, 0x7E00,
                                       0x7C01], np.uint16), rng.integers(0, 0x10000, 5000, dtype=np.uint16)])
    f32 = rng.standard_normal(5000).astype(np.float32)
    for src, dt, exact in ((halves, skv.DTYPE_F16, halves.view(np.float16).astype(np.float32).view(np.uint32)),
                           (halves, skv.DTYPE_BF16, halves.astype(np.uint32) << 16),
                           (f32, skv.DTYPE_FP32, f32.view(np.uint32))):
        n = src.size
        d_src = skv.DeviceBuffer.from_numpy(src)
        d32 = skv.DeviceBuffer(4 * n)
        d16 = skv.DeviceBuffer(2 * n)
        flag = skv.DeviceBuffer.from_numpy(np.zeros(1, np.int32))
        skv.convert_to_f32(d_src, dt, n, d32, flag)
        skv.convert_to_bf16(d_src, dt, n, d16)
        skv.synchronize()
        np.testing.assert_array_equal(d32.download(np.uint32, n), exact)
        np.testing.assert_array_equal(d16.download(np.uint16, n), (exact >> 16).astype(np.uint16))
        has_bad = bool(np.any((exact & 0x7F800000) == 0x7F800000))
        assert bool(flag.download(np.int32, 1)[0]) == has_bad
        flag2 = skv.DeviceBuffer.from_numpy(np.zeros(1, np.int32))
        skv.check_finite(d_src, dt, n, flag2)
        assert bool(flag2.download(np.int32, 1)[0]) == has_bad


@pytest.mark.parametrize("dt", [skv.DTYPE_BF16, skv.DTYPE_F16, skv.DTYPE_FP32])
def test_embedding_lookup(gpu, dt):
    rng = np.random.default_rng(dt)
    vocab, hidden = 300, 2048
    table = (rng.integers(0, 0x7C00, (vocab, hidden), dtype=np.uint16) if dt != skv.DTYPE_FP32
             else rng.standard_normal((vocab, hidden)).astype(np.float32))
    want_rows = {skv.DTYPE_BF16: lambda r: (table[r].astype(np.uint32) << 16).view(np.float32),
                 skv.DTYPE_F16: lambda r: table[r].view(np.float16).astype(np.float32),
                 skv.DTYPE_FP32: lambda r: table[r]}[dt]
    ids = np.array([0, 299, 17, -1, 300], np.int32)
    d_t, d_ids = skv.DeviceBuffer.from_numpy(table), skv.DeviceBuffer.from_numpy(ids)
    out = skv.DeviceBuffer(4 * hidden)
    flags = skv.DeviceBuffer.from_numpy(np.zeros(1, np.int32))
    for i, tok in enumerate(ids):
        skv.embedding(d_t, dt, vocab, hidden, d_ids, i, out, flags)
        got = out.download(np.float32, hidden)
        if 0 <= tok < vocab:
            np.testing.assert_array_equal(got.view(np.uint32), want_rows(tok).view(np.uint32))
        else:
            assert not got.any()
    assert flags.download(np.int32, 1)[0] == skv.FLAG_BAD_TOKEN
    # The rows variant (one launch for a prompt): ids 1.. of the same list.
    rows = skv.DeviceBuffer(4 * hidden * 4)
    flags2 = skv.DeviceBuffer.from_numpy(np.zeros(1, np.int32))
    skv.embedding_rows(d_t, dt, vocab, hidden, d_ids, 1, 4, rows, flags2)
    got = rows.download(np.float32, (4, hidden))
    for r, tok in enumerate(ids[1:]):
        if 0 <= tok < vocab:
            np.testing.assert_array_equal(got[r].view(np.uint32), want_rows(tok).view(np.uint32))
        else:
            assert not got[r].any()
    assert flags2.download(np.int32, 1)[0] == skv.FLAG_BAD_TOKEN


def test_argmax_first_index(gpu):
    rng = np.random.default_rng(9)
    cases = [rng.standard_normal(32000).astype(np.float32), np.zeros(1000, np.float32),
             np.round(rng.standard_normal(32000) * 2).astype(np.float32), -np.abs(rng.standard_normal(7)).astype(np.float32),
             np.full(50000, -3.0, np.float32)]
    cases[1][[5, 900]] = 1.0
    cases[4][[49999, 40000]] = 2.0
    cases.append(np.array([-0.0, 0.0, -0.0], np.float32))
    tail = np.zeros(32003, np.float32)
    tail[[32001, 32002]] = 5.0       # the maximum only in the elements past the last float4
    cases.append(tail)
    ties = np.full(40961, 1.0, np.float32)
    ties[[3, 4, 4099, 40960]] = 7.0  # ties across float4s, batches and the tail
    cases.append(ties)
    want = [osamp.argmax_first(x) for x in cases]
    for shift in (0, 1):             # 16-byte aligned (vector loads) and not (scalar loop)
        ids = skv.DeviceBuffer(4 * len(cases))
        for i, x in enumerate(cases):
            buf = skv.DeviceBuffer.from_numpy(np.concatenate([np.zeros(shift, np.float32), x]))
            skv.lib().skv_argmax_f32(buf.ptr + 4 * shift, x.size, ids.ptr, i, None, None)
        assert list(ids.download(np.int32, len(cases))) == want, f"shift {shift}"


def test_embedding_and_argmax_at_device_index(gpu):
    """skv_embedding_at_f32 / skv_argmax_at_f32 (index and flag word held in
    device memory) give what the host-index calls give."""
    rng = np.random.default_rng(21)
    vocab, hidden = 300, 96
    table = rng.standard_normal((vocab, hidden)).astype(np.float32)
    ids = np.array([5, 17, 299, 1000, 42], np.int32)   # 1000: outside the vocabulary
    d_t, d_ids = skv.DeviceBuffer.from_numpy(table), skv.DeviceBuffer.from_numpy(ids)
    for idx in range(len(ids)):
        state = skv.DeviceBuffer.from_numpy(np.array([idx, 3], np.int32))   # [index, flag word]
        flags = skv.DeviceBuffer.from_numpy(np.zeros(5, np.int32))
        out = skv.DeviceBuffer(4 * hidden)
        gpu._check(skv.lib().skv_embedding_at_f32(d_t.ptr, skv.DTYPE_FP32, vocab, hidden, d_ids.ptr, state.ptr,
                                                  out.ptr, flags.ptr, state.ptr + 4, None))
        ref = skv.DeviceBuffer(4 * hidden)
        ref_flags = skv.DeviceBuffer.from_numpy(np.zeros(1, np.int32))
        skv.embedding(d_t, skv.DTYPE_FP32, vocab, hidden, d_ids, idx, ref, ref_flags)
        np.testing.assert_array_equal(out.download(np.uint32, hidden), ref.download(np.uint32, hidden))
        f = flags.download(np.int32, 5)
        assert f[3] == ref_flags.download(np.int32, 1)[0] and not f[[0, 1, 2, 4]].any()
    logits = rng.standard_normal((4, 32000)).astype(np.float32)
    logits[2, [7, 31999]] = 9.0
    logits[3, 11] = np.nan
    for r in range(4):
        d_l = skv.DeviceBuffer.from_numpy(logits[r])
        out_ids = skv.DeviceBuffer.from_numpy(np.full(8, -1, np.int32))
        state = skv.DeviceBuffer.from_numpy(np.array([r + 2, 1], np.int32))
        flags = skv.DeviceBuffer.from_numpy(np.zeros(3, np.int32))
        gpu._check(skv.lib().skv_argmax_at_f32(d_l.ptr, 32000, out_ids.ptr, state.ptr, flags.ptr, state.ptr + 4,
                                               None))
        ref_ids = skv.DeviceBuffer.from_numpy(np.full(8, -1, np.int32))
        ref_flags = skv.DeviceBuffer.from_numpy(np.zeros(1, np.int32))
        skv.argmax(d_l, 32000, ref_ids, r + 2, ref_flags)
        assert list(out_ids.download(np.int32, 8)) == list(ref_ids.download(np.int32, 8))
        f = flags.download(np.int32, 3)
        assert f[1] == ref_flags.download(np.int32, 1)[0] and f[0] == 0 and f[2] == 0


def _device_sample(logits_row, temp, k, p, u):
    ids = skv.DeviceBuffer.from_numpy(np.zeros(1, np.int32))
    flags = skv.DeviceBuffer.from_numpy(np.zeros(1, np.int32))
    skv.sample(skv.DeviceBuffer.from_numpy(logits_row), logits_row.size, temp, k, p, u, ids, 0, flags)
    return int(ids.download(np.int32, 1)[0]), int(flags.download(np.int32, 1)[0])


SAMPLER_CONFIGS = [(0.0, 0, 1.0), (1.0, 0, 1.0), (0.7, 0, 1.0), (1.0, 1, 1.0), (1.0, 5, 1.0), (1.3, 40, 1.0),
                   (1.0, 0, 0.9), (1.0, 0, 0.5), (0.8, 0, 0.05), (1.0, 50, 0.8), (2.0, 3, 0.99)]


@pytest.mark.parametrize("cfg", SAMPLER_CONFIGS, ids=[f"T{t}-k{k}-p{p}" for t, k, p in SAMPLER_CONFIGS])
def test_sampler_matches_oracle(gpu, cfg):
    temp, k, p = cfg
    rng = np.random.default_rng(abs(hash(cfg)) % 2**32)
    mismatches = 0
    for vocab, rows in ((1000, 24), (32000, 8)):
        logits = rng.standard_normal((rows, vocab)).astype(np.float32) * np.float32(2.0)
        logits[rows // 2:] = np.round(logits[rows // 2:] * 2) / 2    # ties
        us = osamp.canonical_draws(int(rng.integers(0, 2**32)), rows)
        for r in range(rows):
            want, margin = osamp.sample(logits[r], temp, k, p, us[r])
            got, flags = _device_sample(logits[r], temp, k, p, us[r])
            assert flags == 0
            if got != want:
                assert margin < 1e-5, (r, got, want, margin)
                mismatches += 1
    assert mismatches <= 1


def test_sampler_error_flags(gpu):
    x = np.zeros(64, np.float32)
    x[7] = np.nan
    assert _device_sample(x, 1.0, 0, 1.0, 0.5)[1] == skv.FLAG_NONFINITE_LOGITS
    assert _device_sample(x, 0.0, 0, 1.0, 0.5)[1] == skv.FLAG_NONFINITE_LOGITS
    big = np.full(64, 3e38, np.float32)
    assert _device_sample(big, 0.01, 0, 1.0, 0.5)[1] == skv.FLAG_NONFINITE_SCALED
    with pytest.raises(skv.SkvInvalidArgument, match="top_p"):
        _device_sample(np.zeros(8, np.float32), 1.0, 0, 1.5, 0.5)
    with pytest.raises(skv.SkvInvalidArgument, match="temperature"):
        _device_sample(np.zeros(8, np.float32), -1.0, 0, 1.0, 0.5)


# ---------------------------------------------------------------------------
# device loader
# ---------------------------------------------------------------------------
def test_device_loader_values(gpu, tmp_path):
    from test_model_loader import mixed_checkpoint

    path = tmp_path / "mixed.safetensors"
    expected = mixed_checkpoint(path)
    dtypes = {"w.bf16": "BF16", "w.f16": "FP32", "w.f32": "FP32", "model.norm.weight": "FP32"}
    for name, exp in expected.items():
        out = tmp_path / "dump.bin"
        res = tool("load-device", path, "--dump", name, out)
        assert res["ok"] and res["dtype"] == dtypes[name], res
        if res["dtype"] == "BF16":
            np.testing.assert_array_equal(np.fromfile(out, np.uint16), (exp >> 16).astype(np.uint16))
        else:
            np.testing.assert_array_equal(np.fromfile(out, np.uint32), exp)


def test_device_loader_rejects_like_host(gpu, tmp_path):
    from test_model_loader import CASES, write_raw

    for case in ("hole", "dtype_i32", "bad_utf8", "rank_65", "trailing"):
        path = tmp_path / f"{case}.safetensors"
        write_raw(path, *CASES[case])
        host, dev = tool("load-host", path), tool("load-device", path)
        assert not host["ok"] and dev == host


# ---------------------------------------------------------------------------
# Generator against the reference's generations
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def ckpt_dir(tmp_path_factory):
    return str(tmp_path_factory.mktemp("ckpt"))


def _golden(name):
    path = os.path.join(GOLDEN, f"generate_{name}.json")
    if not os.path.exists(path):
        pytest.skip(f"{path} has not been written")
    with open(path) as f:
        return json.load(f)


def _checkpoint(name, ckpt_dir, golden):
    path, sha = make_checkpoint.ensure(name, ckpt_dir)
    assert sha == golden["checkpoint"]["sha256"], "checkpoint writer is not deterministic here"
    return path


def _check_forced(path, golden, n_prompt=None):
    """Teacher-forced logits vs the reference's top-8 per step; returns the
    greedy tokens of the forced run and the max logit error.  n_prompt (default:
    the golden prompt) tokens go through the prompt pass at once; the logits
    from its last row on are checked."""
    prompt, gen = golden["prompt"], golden["generated"]
    tokens = prompt + gen
    n_prompt = len(prompt) if n_prompt is None else n_prompt
    first = n_prompt - len(prompt)   # golden step of the first checked row
    out = os.path.join(os.path.dirname(path), "forced.bin")
    res = tool("forced", path, n_prompt, out, "--", *tokens)
    assert res["ok"], res
    logits = np.fromfile(out, np.float32).reshape(res["rows"], res["vocab"])
    top_ids = np.array(golden["top_ids"])[first:]
    top_vals = np.array(golden["top_vals"], np.float32)[first:]
    assert logits.shape[0] == top_ids.shape[0] == len(tokens) - n_prompt + 1
    got = np.take_along_axis(logits, top_ids, axis=1)
    err = np.abs(got - top_vals)
    bound = LOGIT_ABS + LOGIT_REL * np.abs(top_vals)
    assert (err <= bound).all(), f"max logit error {err.max():.3e} at step {np.unravel_index(err.argmax(), err.shape)}"
    argmax = logits.argmax(axis=1)
    for s, ref_tok in enumerate(top_ids[:, 0]):
        gap = top_vals[s, 0] - top_vals[s, 1]
        if gap > 2 * (LOGIT_ABS + LOGIT_REL * abs(top_vals[s, 0])):
            assert argmax[s] == ref_tok, (s, argmax[s], ref_tok, gap)
    return argmax, float(err.max())


def _check_free_running(tokens, golden):
    """Generated tokens equal the reference CLI's, or diverge first at a step
    where our token is a near-tie in the reference's own logits."""
    want = golden["cli_tokens"]
    if tokens == want:
        return None
    n = min(len(tokens), len(want))
    s = next(i for i in range(n) if tokens[i] != want[i]) if tokens[:n] != want[:n] else n
    step = s - len(golden["prompt"])
    assert 0 <= step < len(golden["top_ids"]), (s, tokens, want)
    ids, vals = golden["top_ids"][step], golden["top_vals"][step]
    assert tokens[s] in ids, f"step {step}: token {tokens[s]} is not in the reference's top-8 {ids}"
    gap = vals[0] - vals[ids.index(tokens[s])]
    assert gap <= 2 * (LOGIT_ABS + LOGIT_REL * abs(vals[0])), (step, gap)
    return step


@pytest.mark.parametrize("loader", ["device", "host"])
def test_generate_mini_matches_reference(gpu, ckpt_dir, loader):
    golden = _golden("mini")
    path = _checkpoint("mini", ckpt_dir, golden)
    extra = ["--host-loader"] if loader == "host" else []
    res = tool("generate", path, len(golden["generated"]), golden["eos"], *extra, "--", *golden["prompt"])
    assert res["ok"], res
    print("mini free-running divergence step:", _check_free_running(res["tokens"], golden))
    assert res["free_blocks"] == 1024 * golden["checkpoint"]["layers"]


def test_forced_logits_mini(gpu, ckpt_dir):
    golden = _golden("mini")
    _, err = _check_forced(_checkpoint("mini", ckpt_dir, golden), golden)
    print(f"mini max logit error {err:.3e}")


def test_generate_repeatable_and_errors(gpu, ckpt_dir):
    golden = _golden("mini")
    path = _checkpoint("mini", ckpt_dir, golden)
    prompt = golden["prompt"]
    base = tool("generate", path, 40, -1, "--", *prompt)
    res = tool("generate", path, 40, -1, "--repeat", 3, "--", *prompt)
    assert base["ok"] and res["ok"] and len(res["gen_ms"]) == 3
    assert res["tokens"] == base["tokens"] and len(base["tokens"]) == 56
    bad = tool("generate", path, 4, -1, "--", 5, 1000)
    assert bad == {"ok": False, "error": "Generator: prompt token outside vocabulary"}
    big = tool("generate", path, 1024 * 16, -1, "--", 5)
    assert big == {"ok": False, "error": "Generator: prompt plus max exceeds KV capacity"}
    # EOS: generation stops right after the first EOS, which is kept; with the
    # device loop running ahead, later queued steps must not leak into the result.
    gen = base["tokens"][16:]
    for pick in (0, 5, 30):
        eos = gen[pick]
        first = gen.index(eos)
        res = tool("generate", path, 40, eos, "--", *prompt)
        assert res["tokens"] == prompt + gen[: first + 1], (pick, eos)
        assert res["free_blocks"] == 1024 * golden["checkpoint"]["layers"]
    # a prompt ending in EOS is returned as is
    res = tool("generate", path, 40, gen[0], "--", 3, gen[0])
    assert res["tokens"] == [3, gen[0]]


def _parity_run(path, max_new, prompt):
    env = dict(os.environ, STRATAKV_PARITY="1")
    p = subprocess.run([TOOL, "generate", path, str(max_new), "-1", "--", *map(str, prompt)], stdout=subprocess.PIPE,
                       stderr=subprocess.PIPE, text=True, timeout=600, env=env)
    res = json.loads(p.stdout.strip().splitlines()[-1])
    assert p.returncode == 0 and res["ok"], p.stderr
    lines = p.stderr.splitlines()
    ops = {}
    for line in lines:
        if line.startswith("[PARITY L0] "):
            name, rest = line[len("[PARITY L0] "):].split(": max_diff = ")
            ops[name] = float(rest.split(",")[0])
    layers = {}
    for line in lines:
        if line.startswith("[PARITY pos=") and " layer=" in line:
            head, val = line.split("] max_diff = ")
            pos, layer = head[len("[PARITY pos="):].split(" layer=")
            layers[(int(pos), int(layer))] = float(val)
    final = [line for line in lines if line.startswith("[PARITY FINAL] lm_head logits")]
    return res, ops, layers, final


@pytest.mark.parametrize("prompt_len", [1, 3])
def test_parity_diagnostic_reports_every_layer(gpu, ckpt_dir, prompt_len):
    """STRATAKV_PARITY=1 (src/generation/generator.cpp:33-36, 581-613): every
    layer at every position against the host model of the layer, in the
    reference's line format.
    * layer 0's ops on the first token (the values the fused kernels leave in
      memory), the embedding bit-exact;
    * one line per position and layer, for the prompt (one step, or the
      prompt pass over 3 rows) and every decode step that ran;
    * the final logits the first token is chosen from, same argmax.
    The host model keeps K/V rounded to bf16 like the pools, so the
    differences are the fp32 arithmetic's: bounded here by 1e-3 of the
    values' scale (a dropped term or a wrong position errs by O(1))."""
    golden = _golden("mini")
    path = _checkpoint("mini", ckpt_dir, golden)
    prompt = golden["prompt"][:prompt_len]
    res, ops, layers, final = _parity_run(path, 4, prompt)
    L = golden["checkpoint"]["layers"]
    assert set(ops) == {"embedding", "rope_q", "rope_k", "v_proj", "paged_attention", "out_proj + residual",
                        "swiglu"}, ops
    assert ops["embedding"] == 0.0, ops
    assert max(ops.values()) < 1e-3, ops
    positions = len(res["tokens"]) - 1        # the prompt and every generated token but the last
    assert sorted(layers) == [(p, l) for p in range(positions) for l in range(L)], sorted(layers)
    assert max(layers.values()) < 1e-3, layers
    assert len(final) == 1, final
    ga, ca = (int(final[0].split(name + " = ")[1].split(",")[0]) for name in ("gpu_argmax", "cpu_argmax"))
    assert ga == ca, final[0]
    # The diagnostic turns graph replay off; the tokens are those of a plain run.
    plain = tool("generate", path, 4, -1, "--", *prompt)
    assert res["tokens"] == plain["tokens"]


def test_generate_leaves_the_pools_unchanged(gpu, ckpt_dir):
    """The reference's SequenceGuard puts every pool back after generate
    (src/generation/generator.cpp:347-371, 639): with every K/V pool filled
    with random bf16 first, the pools hash the same after each of two
    generations (graph replay and step by step), and the attention of the
    last step read the blocks of the whole context."""
    golden = _golden("mini")
    path = _checkpoint("mini", ckpt_dir, golden)
    prompt = golden["prompt"]
    for extra in ([], ["--eager"]):
        res = tool("generate", path, 40, -1, "--check-pools", "--repeat", 2, *extra, "--", *prompt)
        assert res["ok"], res
        assert res["pools_unchanged"] == [1, 1], res
        positions = len(res["tokens"]) - 1
        want = -(-positions // 16)
        # Replayed steps leave the count of the prompt's prefill_into / forward_into.
        assert res["blocks_visited"][1] == (-(-len(prompt) // 16) if res["replayed"][1] else want), res
        assert res["replayed"][1] == (0 if extra else res["replayed"][1])


def test_consecutive_generations_use_the_same_blocks(gpu, ckpt_dir):
    """The reference restores every layer's pool after generate (SequenceGuard,
    src/generation/generator.cpp:347-371), so each generation on a fresh
    Generator allocates exactly as a fresh pool would: the table of
    allocate_sequence + one append_token per position that is processed (the
    prompt and every generated token but the last), on the oracle's
    restatement of BlockPool / PageTable, twice in a row."""
    from oracle import OP_ALLOC_SEQ, OP_APPEND
    golden = _golden("mini")
    path = _checkpoint("mini", ckpt_dir, golden)
    prompt = golden["prompt"]
    res = tool("generate", path, 40, -1, "--repeat", 3, "--", *prompt)
    assert res["ok"], res
    n_appends = len(res["tokens"]) - 1
    ops = [(OP_ALLOC_SEQ, 0)] + [(OP_APPEND, 0)] * n_appends
    _, lens, blocks, _ = oracle.pool_trace(1024, 16, ops, 1, 64)
    want = blocks[0, : -(-int(lens[0]) // 16)].tolist()
    assert res["tables"] == [want, want, want], (res["tables"], want)
    assert res["free_blocks"] == 1024 * golden["checkpoint"]["layers"]


def test_sampled_generate_stops_the_stream_at_eos(gpu, ckpt_dir):
    """Sampling draws once per generated step, up to and including the EOS
    step, as the reference's loop does (src/generation/generator.cpp:717-788):
    the host queues steps ahead of the device, and the draws it made for steps
    past the EOS are taken back.  A generator that stops at EOS after e + 1
    tokens and one whose first call asks for exactly e + 1 tokens (no EOS) must
    then produce the same second generation from the same seed."""
    golden = _golden("mini")
    path = _checkpoint("mini", ckpt_dir, golden)
    prompt = golden["prompt"]
    base = tool("generate", path, 40, -1, "--temp", 1.0, "--seed", 7, "--", *prompt)
    assert base["ok"], base
    gen = base["tokens"][len(prompt):]
    for pick in (2, 11):
        eos = gen[pick]
        e = gen.index(eos)  # first occurrence: the EOS step
        stopped = tool("generate", path, 40, eos, "--temp", 1.0, "--seed", 7, "--repeat", 2, "--", *prompt)
        exact = tool("generate", path, 40, eos, "--temp", 1.0, "--seed", 7, "--repeat", 2, "--first-max", e + 1,
                     "--", *prompt)
        assert stopped["ok"] and exact["ok"]
        assert stopped["runs"][0] == exact["runs"][0] == prompt + gen[: e + 1], (pick, e)
        assert stopped["runs"][1] == exact["runs"][1], (pick, e, stopped["runs"][1], exact["runs"][1])


@pytest.mark.timeout(400)  # writes a 2.2 GB checkpoint first (~30 s on 8 cores)
def test_generate_tinyllama_matches_reference(gpu, ckpt_dir):
    golden = _golden("tinyllama")
    path = _checkpoint("tinyllama", ckpt_dir, golden)
    res = tool("generate", path, len(golden["generated"]), golden["eos"], "--", *golden["prompt"])
    assert res["ok"], res
    print("tinyllama free-running divergence step:", _check_free_running(res["tokens"], golden),
          "gen_ms", res["gen_ms"], "load_ms", res["load_ms"])
    _, err = _check_forced(path, golden)
    print(f"tinyllama max logit error {err:.3e}")
    # A 100-token prompt (the projections of the prompt pass on the matrix
    # cores, inputs split into hi + lo bf16 parts), then the 44 remaining
    # tokens teacher-forced through the cache it wrote: the same bounds.
    _, err = _check_forced(path, golden, n_prompt=100)
    print(f"tinyllama max logit error after a 100-token prompt pass {err:.3e}")


# ---------------------------------------------------------------------------
# Decode steps replayed from a HIP graph against step-by-step launches
# ---------------------------------------------------------------------------
def _small(ckpt_dir):
    path, _ = make_checkpoint.ensure("small", ckpt_dir)
    return path


@pytest.mark.parametrize("max_new", [2, 40, 240])
def test_graph_replay_matches_eager(gpu, ckpt_dir, max_new):
    """Generations whose steps are replayed from one captured graph give the
    tokens, block tables and last logits (bits) of the same generations
    launched step by step, over three generations in a row (the graph is
    recorded once and reused).  240 new tokens fill the 16-block short-table
    limit exactly (16 + 240 = 256)."""
    path = _small(ckpt_dir)
    prompt = [3, 141, 59, 265, 358, 979, 323, 846, 264, 338, 327, 950, 288, 419, 716, 939]
    g = tool("generate", path, max_new, -1, "--repeat", 3, "--", *prompt)
    e = tool("generate", path, max_new, -1, "--repeat", 3, "--eager", "--", *prompt)
    assert g["ok"] and e["ok"], (g, e)
    assert g["replayed"] == [1, 1, 1] and e["replayed"] == [0, 0, 0]
    assert g["runs"] == e["runs"] and len(g["tokens"]) == 16 + max_new
    assert g["runs"][0] == g["runs"][1] == g["runs"][2]
    assert g["tables"] == e["tables"]
    assert g["logits_fnv"] == e["logits_fnv"] and len(set(g["logits_fnv"])) == 1


def test_graph_replay_past_the_short_table_limit_runs_eagerly(gpu, ckpt_dir):
    path = _small(ckpt_dir)
    g = tool("generate", path, 241, -1, "--", *range(1, 17))   # 257 tokens: 17 blocks
    assert g["ok"] and g["replayed"] == [0]


def test_graph_replay_eos_and_sampling(gpu, ckpt_dir):
    """EOS in the middle of a replayed generation, and sampled generations
    (the draws stay launches of their own before each replayed step): the same
    tokens, tables and flags behaviour as step-by-step launches."""
    path = _small(ckpt_dir)
    prompt = [11, 22, 33, 44, 55]
    base = tool("generate", path, 60, -1, "--eager", "--", *prompt)
    assert base["ok"]
    # A token chosen at step 20 or later (and not in the prompt) ends the
    # generation at its first occurrence.
    eos = next(t for t in base["tokens"][len(prompt) + 20:] if t not in prompt)
    first = base["tokens"].index(eos, len(prompt))
    for extra in ([], ["--eager"]):
        r = tool("generate", path, 60, eos, *extra, "--", *prompt)
        assert r["ok"] and r["tokens"] == base["tokens"][:first + 1], (extra, r)
    runs = {}
    for extra in ([], ["--eager"]):
        r = tool("generate", path, 50, -1, "--temp", 0.9, "--top-k", 20, "--top-p", 0.95, "--seed", 7,
                 "--repeat", 2, *extra, "--", *prompt)
        assert r["ok"], r
        runs[bool(extra)] = r
    assert runs[False]["replayed"] == [1, 1] and runs[True]["replayed"] == [0, 0]
    assert runs[False]["runs"] == runs[True]["runs"]
    assert runs[False]["logits_fnv"] == runs[True]["logits_fnv"]
