"""skv_paged_block_checksum (the decode's load pattern with the math replaced
by a checksum, used by bench.py --load-calibration) against numpy.

checksums[b * Hkv + h] = wrapping uint32 sum of the 32-bit words of the head-h
slice of every row of K and V in the first min(ceil(L_b / 16), max_blocks)
table entries of sequence b; entries outside the pool add 0.  Exact (integer),
so every block must be read exactly once whatever the grid split: ragged and
empty sequences, lengths past the table, invalid entries, one sequence split
over many wavefronts and many short sequences per wavefront.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def expected(k, v, tables, lens, Hkv, bs=16):
    total = k.shape[0]
    kw = k.view(np.uint32).reshape(total, bs, Hkv, -1).astype(np.uint64)
    vw = v.view(np.uint32).reshape(total, bs, Hkv, -1).astype(np.uint64)
    per_block = kw.sum(axis=(1, 3)) + vw.sum(axis=(1, 3))  # [total, Hkv]
    out = np.zeros((len(lens), Hkv), np.uint64)
    for b, L in enumerate(lens):
        nb = min(-(-int(L) // bs), tables.shape[1]) if L > 0 else 0
        ids = tables[b, :nb]
        ids = ids[(ids >= 0) & (ids < total)]
        out[b] = per_block[ids].sum(axis=0)
    return (out & 0xFFFFFFFF).astype(np.uint32).reshape(-1)


def run(skv, Hq, Hkv, hd, lens, max_blocks, total, seed, bad_entries=0):
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    B = len(lens)
    k = rng.integers(0, 1 << 16, size=(total, 16, Hkv, hd), dtype=np.uint16)
    v = rng.integers(0, 1 << 16, size=(total, 16, Hkv, hd), dtype=np.uint16)
    perm = rng.permutation(total).astype(np.int32)
    tables = np.resize(perm, (B, max_blocks)).astype(np.int32)
    for _ in range(bad_entries):  # entries outside the pool read as zeros
        b, j = rng.integers(0, B), rng.integers(0, max_blocks)
        tables[b, j] = int(rng.choice([-1, -7, total, total + 100]))
    d_k, d_v = skv.DeviceBuffer.from_numpy(k), skv.DeviceBuffer.from_numpy(v)
    d_t, d_l = skv.DeviceBuffer.from_numpy(tables), skv.DeviceBuffer.from_numpy(lens)
    sums = skv.DeviceBuffer(B * Hkv * 4)
    skv.paged_block_checksum(d_k, d_v, total, d_t, max_blocks, d_l, B, Hq, Hkv, hd, 16, sums)
    skv.synchronize()
    got = sums.download(np.uint32, (B * Hkv,))
    want = expected(k, v, tables, lens, Hkv)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} of {B * Hkv} checksums differ, first (seq, head) " \
                          f"{divmod(int(bad[0]), Hkv)}: {got[bad[0]]:#x} != {want[bad[0]]:#x}"


@pytest.mark.parametrize("Hq,Hkv,hd", [(32, 8, 128), (32, 4, 64), (16, 2, 64), (16, 1, 128), (8, 8, 64)],
                         ids=["l3", "tl", "wpw2", "wpw1", "mha"])
def test_ragged_batch(gpu, Hq, Hkv, hd):
    rng = np.random.default_rng(Hq * 100 + Hkv)
    lens = rng.integers(0, 3000, size=37)
    lens[:4] = [0, 1, 16, 17]
    run(gpu, Hq, Hkv, hd, lens, max_blocks=190, total=1500, seed=Hkv, bad_entries=20)


def test_one_long_sequence_split_over_the_grid(gpu):
    # 4,097 tokens = 257 blocks over many stream-K ranges of one sequence.
    run(gpu, 32, 4, 64, [4097], max_blocks=300, total=600, seed=5)


def test_lengths_past_the_table(gpu):
    # Lengths beyond max_blocks * 16 read only the table's blocks.
    run(gpu, 32, 8, 128, [5000, 100, 2000], max_blocks=40, total=200, seed=6)


def test_many_short_sequences(gpu):
    lens = np.random.default_rng(9).integers(1, 80, size=700)
    run(gpu, 32, 4, 64, lens, max_blocks=5, total=4000, seed=9, bad_entries=50)


@pytest.mark.parametrize("B", [64, 2000])
def test_short_and_empty_segments_ranges_among_segment_slots(gpu, B):
    # The split charges every non-empty segment a few empty slots before its
    # blocks: with 1-5 block segments and a fifth of the sequences empty,
    # range boundaries fall among those slots (at B=64 the ranges are 4 slots
    # wide, some hold no block); every block is still read exactly once.
    rng = np.random.default_rng(B)
    lens = rng.integers(1, 80, size=B)
    lens[rng.random(B) < 0.2] = 0
    run(gpu, 32, 4, 64, lens, max_blocks=25, total=6000, seed=B, bad_entries=B // 20)


def test_rejects_other_geometries(gpu):
    skv = gpu
    buf = skv.DeviceBuffer(1 << 16)
    t = skv.DeviceBuffer.from_numpy(np.zeros((1, 4), np.int32))
    lens = skv.DeviceBuffer.from_numpy(np.array([5], np.int32))
    with pytest.raises(skv.SkvError):  # block_size 8
        skv.paged_block_checksum(buf, buf, 4, t, 4, lens, 1, 8, 8, 64, 8, buf)
    with pytest.raises(skv.SkvError):  # head_dim 96
        skv.paged_block_checksum(buf, buf, 4, t, 4, lens, 1, 8, 8, 96, 16, buf)
    with pytest.raises(skv.SkvError):  # group 3
        skv.paged_block_checksum(buf, buf, 4, t, 4, lens, 1, 12, 4, 64, 16, buf)


# ---------------------------------------------------------------------------
# skv_stream_read_checksum (bench.py --read-calibration): the wrapping uint32
# sum of a buffer's 32-bit words, so every 16-byte piece must be read exactly
# once: sizes below one wave-wide load, not a multiple of the unrolled step,
# spanning several 4 MiB chunks and more chunks than the grid has wavefronts.
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("nbytes", [16, 1008, 4 << 20, (4 << 20) + 48, (37 << 20) + 4096 + 16],
                         ids=["one_piece", "partial_step", "one_chunk", "chunk_plus", "many_chunks"])
def test_stream_read_checksum(gpu, nbytes):
    skv = gpu
    rng = np.random.default_rng(nbytes % 1000)
    words = rng.integers(0, 1 << 32, size=nbytes // 4, dtype=np.uint32)
    d = skv.DeviceBuffer.from_numpy(words)
    out = skv.DeviceBuffer(4)
    skv.stream_read_checksum(d, nbytes, out)
    skv.synchronize()
    got = int(out.download(np.uint32, (1,))[0])
    assert got == int(words.astype(np.uint64).sum() & 0xFFFFFFFF)


def test_stream_read_checksum_repeated_calls(gpu):
    # Each call clears the sum before reading: two calls in a row give the
    # word count of a buffer of ones (5 chunks and a 16-byte tail), not twice it.
    skv = gpu
    nbytes = (4 << 20) * 5 + 16
    d = skv.DeviceBuffer.from_numpy(np.ones(nbytes // 4, np.uint32))
    out = skv.DeviceBuffer(4)
    for _ in range(2):
        skv.stream_read_checksum(d, nbytes, out)
    skv.synchronize()
    assert int(out.download(np.uint32, (1,))[0]) == nbytes // 4


def test_stream_read_checksum_rejects(gpu):
    skv = gpu
    buf = skv.DeviceBuffer(1 << 12)
    out = skv.DeviceBuffer(4)
    with pytest.raises(skv.SkvError):
        skv.stream_read_checksum(buf, 24, out)   # not a multiple of 16
    with pytest.raises(skv.SkvError):
        skv.stream_read_checksum(buf, 0, out)
