"""Order- and stream-level pins of the oracle (oracle/oracle.cpp).

Each test below has an answer fixed by IEEE binary32/binary64 arithmetic and
the operation order the reference's source states, or by a published test
vector, chosen so that a plausible restatement slip gives a different answer:

- the pairwise lane reduce of distance.rs:534-538, the lane assignment of
  chunks_exact(8) and the separate sequential tail (distance.rs:267-283,
  317-331): 2^24 + 1 rounds back to 2^24 (ties to even), so the order in which
  the 1s meet 2^24 decides between 16777216 and 16777218;
- the *sequential* sums of k-means `squared` (kmeans.rs:234-241), of the PQ
  table loop (product.rs:416-433) and of PQ `nearest_centroid`, against the
  *unrolled* kernel of IVF `nearest_centroid` (ivfpq.rs:1231-1243);
- the NaN a cancelling overflow produces, its sign on the reference's aarch64
  platform, and where total_cmp ranks it (topk.rs:63-67);
- the rand 0.8 samplers against the raw ChaCha stream (kmeans.rs:150, 167-169;
  fixture.rs:120-121), rand_core's seed_from_u64 against the published PCG32
  generator, and the ChaCha core at 8 and 12 rounds against published vectors.

test_planted_mistakes_are_caught compiles mutated copies of oracle.cpp and
checks that these tests, and the composition pins of
test_oracle_compositions.py, fail on each.
"""
import os
import re
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from oracle import oracle as orc

F32_MAX = np.float32(3.4028235e38)
TWO24 = 16777216.0


def bits(x):
    return int(np.float32(x).view(np.uint32))


def f32v(*xs):
    return np.array(xs, np.float32)


# --- distance.rs:267-283, 317-331, 534-538 -------------------------------------------
def test_kat_pairwise_reduce():
    z = np.zeros(8, np.float32)
    # squares [2^24, 1, 1, 1, 0, 0, 0, 0]: ((2^24+1)+(1+1)) + 0 = 2^24 + 2;
    # one at a time, every 1 rounds away: 2^24
    v = f32v(4096, 1, 1, 1, 0, 0, 0, 0)
    assert orc.squared_euclidean(v, z) == TWO24 + 2
    assert orc.squared_euclidean_scalar(v, z) == TWO24
    assert orc.dot(v, v) == TWO24 + 2
    assert orc.dot_scalar(v, v) == TWO24
    assert orc.manhattan(f32v(TWO24, 1, 1, 1, 0, 0, 0, 0), z) == TWO24 + 2
    # the same in lanes 4..7 (the second half of the tree)
    assert orc.squared_euclidean(f32v(0, 0, 0, 0, 4096, 1, 1, 1), z) == TWO24 + 2
    # squares [2^24, 1, 0, 1]: (0+1)+(2+3) = 2^24 + 1 -> 2^24, while a
    # (0+2)+(1+3) pairing would give 2^24 + 2
    assert orc.squared_euclidean(f32v(4096, 1, 0, 1, 0, 0, 0, 0), z) == TWO24
    # the two halves meet last: [2^24,0,0,0 | 1,0,1,0] -> 2^24 + 2
    assert orc.squared_euclidean(f32v(4096, 0, 0, 0, 1, 0, 1, 0), z) == TWO24 + 2


def test_kat_lane_of_each_element():
    # chunks_exact(8): element i accumulates into lane i % 8. With the 1s of the
    # second chunk in lanes 1..3 the sum is 2^24 + 2; in lanes 0..2 the first
    # 1 meets 2^24 alone and rounds away (2^24); contiguous blocks of two
    # elements per lane would give lanes [2^24,0,0,0,1,2,0,0] -> 2^24 + 4
    a = np.zeros(16, np.float32)
    a[0] = 4096
    a[9:12] = 1
    assert orc.squared_euclidean(a, np.zeros(16, np.float32)) == TWO24 + 2
    a = np.zeros(16, np.float32)
    a[0] = 4096
    a[8:11] = 1
    assert orc.squared_euclidean(a, np.zeros(16, np.float32)) == TWO24


def test_kat_tail_is_summed_apart_then_added():
    # dim 10: lanes [2^24, 0...], tail = 1 + 1 = 2, total 2^24 + 2. Adding
    # the tail elements one by one to the reduced sum, or into lanes 0 and 1,
    # would give 2^24.
    a = np.zeros(10, np.float32)
    a[0] = 4096
    a[8:10] = 1
    assert orc.squared_euclidean(a, np.zeros(10, np.float32)) == TWO24 + 2
    assert orc.dot(a, a) == TWO24 + 2


def test_kat_cancelling_overflow_is_a_positive_nan():
    a = f32v(F32_MAX, F32_MAX, F32_MAX, F32_MAX, 0, 0, 0, 0)
    b = f32v(1, 1, -1, -1, 0, 0, 0, 0)
    # (MAX+MAX) + (-MAX-MAX) = inf + -inf: NaN. Sequentially: +inf. A
    # (0+2)+(1+3) pairing: 0.
    d = orc.dot(a, b)
    assert np.isnan(d)
    assert orc.dot_scalar(a, b) == np.inf
    # aarch64's default NaN has its sign clear; inner_product negates it
    assert bits(d) == 0x7FC00000
    assert bits(orc.space_distance(orc.INNER_PRODUCT, a, b)) == 0xFFC00000
    assert bits(orc.space_distance(orc.COSINE, a, b)) == 0x7FC00000
    assert bits(orc.metric_distance(orc.INNER_PRODUCT, a, b)) == 0xFFC00000


def test_kat_nan_scores_rank_by_total_cmp():
    # topk.rs:63-67: -NaN sorts before every number, +NaN after every number.
    # An inner-product search whose query cancels a stored vector's overflow
    # ranks that vector first; cosine (1 - NaN = +NaN) ranks it last.
    data = np.array([[1, 0, 0, 0, 0, 0, 0, 0],
                     [F32_MAX] * 8,
                     [0, 1, 0, 0, 0, 0, 0, 0],
                     [0, 0, 0, 0, 2, 0, 0, 0]], np.float32)
    ids = np.array([10, 11, 12, 13], np.uint64)
    q = f32v(1, 1, 1, 1, -1, -1, -1, -1)
    oi, od, oc = orc.flat_search(orc.prepare_rows(orc.INNER_PRODUCT, data), ids, orc.INNER_PRODUCT,
                                 q.reshape(1, 8), 4)
    assert list(oi[0]) == [11, 10, 12, 13]
    assert bits(od[0, 0]) == 0xFFC00000
    assert list(od[0, 1:]) == [-1.0, -1.0, 2.0]
    pd = orc.prepare_rows(orc.COSINE, data)
    assert np.array_equal(pd[1], data[1])  # |x| overflows: normalize_in_place leaves it
    oi, od, oc = orc.flat_search(pd, ids, orc.COSINE, orc.prepare_rows(orc.COSINE, q.reshape(1, 8)), 4)
    assert oi[0, -1] == 11 and bits(od[0, -1]) == 0x7FC00000


# --- sequential sums: kmeans.rs:234-241, product.rs:416-433 / 463-515 vs ivfpq.rs:1231-1243 ----
V = f32v(4096, 1, 1, 1, 0, 0, 0, 0)
# V - B = [4096, 1.25, 0, ...]: 2^24 + 1.5625 rounds to 2^24 + 2 in either order
B = f32v(0, -0.25, 1, 1, 0, 0, 0, 0)
A = np.zeros(8, np.float32)  # |V - A|^2: 2^24 sequentially, 2^24 + 2 pairwise


def test_kat_kmeans_squared_is_sequential():
    a, d = orc.kmeans_assign(V.reshape(1, 8), np.stack([B, A]))
    # sequential: A at 2^24 beats B at 2^24 + 2; pairwise they would tie and
    # the strict < would keep B (index 0)
    assert int(a[0]) == 1 and float(d[0]) == TWO24
    cents, assign, inertia, iters = orc.kmeans_lloyd(V.reshape(1, 8), np.stack([B, A]), 1)
    assert int(assign[0]) == 1 and inertia == TWO24


def _books(rows):
    books = np.full((256, 8), 1e6, np.float32)
    books[: len(rows)] = rows
    return books.reshape(-1)


def test_kat_pq_table_and_encode_are_sequential():
    sq, dt = orc.pq_table(_books([A, V]), 8, 1, V)
    assert sq[0] == TWO24  # sum of (V - 0)^2 in dimension order
    assert dt[1] == TWO24  # V . V in dimension order
    # nearest_centroid: sequential sum, strict <
    codes = orc.pq_encode(_books([B, A]), 8, 1, V.reshape(1, 8))
    assert int(codes[0, 0]) == 1


def test_kat_ivf_nearest_centroid_is_unrolled():
    # ivfpq.rs:1231-1243 scores lists with squared_euclidean_unrolled: both
    # lists at 2^24 + 2, so the strict < keeps list 0
    codes, list_of = orc.ivf_encode(V.reshape(1, 8), np.stack([B, A]), _books([A]), 1)
    assert int(list_of[0]) == 0
    # the residual V - B = [4096, 1.25, 0...] is nearest codebook row 0 (A)
    assert int(codes[0, 0]) == 0


# --- rand 0.8 / rand_chacha 0.3 / rand_core 0.6 at the stream level ---------------------------
def _twins(seed):
    return orc.Rng(seed), orc.Rng(seed)


def test_kat_gen_range_power_of_two_takes_the_high_bits():
    # UniformInt::sample_single with range 2^j: the widening multiply's high
    # word is v >> (64 - j); the conservative zone (range << lz) - 1 = 2^63 - 1
    # accepts v iff bit 63 - j of v is clear. v % 2^j would take the low bits.
    for seed in (1, 0x9E3779B9):
        raw, smp = _twins(seed)
        for j in (1, 2, 5, 11, 17, 21, 32, 40, 63):
            while True:
                v = raw.next_u64()
                if not (v >> (63 - j)) & 1:
                    break
            assert smp.gen_range_usize(1 << j) == v >> (64 - j), (seed, j)
        assert raw.next_u32() == smp.next_u32()  # the same number of draws


def test_kat_gen_range_f64_is_52_high_bits_times_scale():
    # UniformFloat<f64>::sample_single(0, total): the top 52 bits as a
    # mantissa in [1, 2), minus 1, times the scale, plus 0.
    raw, smp = _twins(7)
    for total in (1.0, 3.5, 12345.678, 2.0 ** 40 + 3):
        for _ in range(200):
            v = raw.next_u64()
            want = (float(v >> 12) * 2.0 ** -52) * total
            assert smp.gen_range_f64(0.0, total) == want


def test_kat_gen_f32_is_24_high_bits():
    raw, smp = _twins(11)
    for _ in range(500):
        u = raw.next_u32()
        assert smp.gen_f32() == np.float32((u >> 8) * 2.0 ** -24)


def test_kat_next_u64_straddles_a_refill():
    # rand_core BlockRng::next_u64 at index 63: the last word of the buffer is
    # the low half, the first word of the next four blocks the high half
    r = orc.Rng(3)
    key = r.key()
    w = np.concatenate([orc.chacha_block(key, c, 0, 8) for c in range(8)])
    for _ in range(63):
        r.next_u32()
    assert r.next_u64() == (int(w[64]) << 32) | int(w[63])
    assert r.next_u32() == int(w[65])


M64 = (1 << 64) - 1
PCG_MUL = 6364136223846793005


def _pcg32(state, inc, n):
    """The published PCG32 generator (pcg_basic.c, pcg32_random_r): output
    from the old state by XSH-RR, then advance with the LCG."""
    out = []
    for _ in range(n):
        old = state
        state = (old * PCG_MUL + inc) & M64
        xs = (((old >> 18) ^ old) >> 27) & 0xFFFFFFFF
        rot = old >> 59
        out.append(((xs >> rot) | (xs << ((-rot) & 31))) & 0xFFFFFFFF)
    return out


def test_pcg32_matches_the_published_demo_vector():
    # pcg32_srandom_r(42, 54): state 0, inc 2*54+1, one step, add 42, one step;
    # the first six outputs printed by pcg32-demo
    inc = (54 << 1) | 1
    state = (0 * PCG_MUL + inc) & M64
    state = (state + 42) & M64
    state = (state * PCG_MUL + inc) & M64
    assert _pcg32(state, inc, 6) == [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293, 0xBFA4784B, 0xCBED606E]


def test_kat_seed_from_u64_is_pcg32():
    # rand_core 0.6 seed_from_u64: advance (MUL, INC = 11634580027462260723)
    # first, then output from the new state, eight times -> the 32-byte key.
    # That is the PCG32 stream started one step in.
    inc = 11634580027462260723
    for seed in (0, 1, 42, 0x1FF9C0D, 0x5EED1EAF, 0x9E3779B9, M64):
        want = _pcg32((seed * PCG_MUL + inc) & M64, inc, 8)
        assert [int(x) for x in orc.Rng(seed).key()] == want, hex(seed)


def _le_hex(words):
    return b"".join(int(w).to_bytes(4, "little") for w in words).hex()


def test_chacha_8_and_12_rounds_match_published_vectors():
    # draft-strombergson-chacha-test-vectors, TC1 (all-zero 256-bit key and
    # 64-bit IV, block 0) for 8 and 12 rounds; RFC 7539 A.1 pins 20 rounds
    z = np.zeros(8, np.uint32)
    assert _le_hex(orc.chacha_block(z, 0, 0, 8)) == (
        "3e00ef2f895f40d67f5bb8e81f09a5a12c840ec3ce9a7f3b181be188ef711a1e"
        "984ce172b9216f419f445367456d5619314a42a3da86b001387bfdb80e0cfe42")
    assert _le_hex(orc.chacha_block(z, 0, 0, 12)) == (
        "9bf49a6a0755f953811fce125f2683d50429c3bb49e074147e0089a52eae155f"
        "0564f879d27ae3c02ce82834acfa8c793a629f2ca0de6919610be82f411326be")


# --- planted mistakes ---------------------------------------------------------------------
# (name, text in oracle.cpp, replacement, tests of this file that must fail)
MUTANTS = [
    ("sequential lane reduce",
     "  float a = (acc[0] + acc[1]) + (acc[2] + acc[3]);\n  float b = (acc[4] + acc[5]) + (acc[6] + acc[7]);\n  return a + b;",
     "  float s = acc[0];\n  for (size_t j = 1; j < LANES; ++j) s += acc[j];\n  return s;",
     ["test_kat_pairwise_reduce", "test_kat_cancelling_overflow_is_a_positive_nan", "test_kat_ivf_nearest_centroid_is_unrolled"]),
    ("(0+2)+(1+3) pairing",
     "  float a = (acc[0] + acc[1]) + (acc[2] + acc[3]);",
     "  float a = (acc[0] + acc[2]) + (acc[1] + acc[3]);",
     ["test_kat_pairwise_reduce", "test_kat_cancelling_overflow_is_a_positive_nan"]),
    ("tail folded into the lanes",
     "  float tail = 0.0f;\n  for (size_t i = chunks * LANES; i < n; ++i) {\n    float d = a[i] - b[i];\n    tail += d * d;\n  }\n  return reduce8(acc) + tail;",
     "  for (size_t i = chunks * LANES; i < n; ++i) {\n    float d = a[i] - b[i];\n    acc[i - chunks * LANES] += d * d;\n  }\n  return reduce8(acc);",
     ["test_kat_tail_is_summed_apart_then_added"]),
    ("k-means squared unrolled",
     "inline float km_squared(const float* a, const float* b, size_t n) { return sq_l2_scalar(a, b, n); }",
     "inline float km_squared(const float* a, const float* b, size_t n) { return sq_l2_unrolled(a, b, n); }",
     ["test_kat_kmeans_squared_is_sequential"]),
    ("x86 NaN sign",
     "inline float arm_nan(float x) { return std::isnan(x) ? std::numeric_limits<float>::quiet_NaN() : x; }",
     "inline float arm_nan(float x) { return std::isnan(x) ? -std::numeric_limits<float>::quiet_NaN() : x; }",
     ["test_kat_cancelling_overflow_is_a_positive_nan", "test_kat_nan_scores_rank_by_total_cmp"]),
    ("gen_range by modulo",
     "      if (lo <= zone) return hi;",
     "      (void)hi; (void)lo; (void)zone; return v % range;",
     ["test_kat_gen_range_power_of_two_takes_the_high_bits"]),
    ("gen_range_f64 from the low bits",
     "      uint64_t bits = (next_u64() >> 12) | (uint64_t(1023) << 52);",
     "      uint64_t bits = (next_u64() & ((uint64_t(1) << 52) - 1)) | (uint64_t(1023) << 52);",
     ["test_kat_gen_range_f64_is_52_high_bits_times_scale"]),
    ("gen_f32 from the low bits",
     "  float gen_f32() { return (float)(next_u32() >> 8) * (1.0f / 16777216.0f); }",
     "  float gen_f32() { return (float)(next_u32() & 0xFFFFFFu) * (1.0f / 16777216.0f); }",
     ["test_kat_gen_f32_is_24_high_bits"]),
    ("seed_from_u64 outputs the old state",
     "    state = state * MUL + INC;\n    uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);\n    uint32_t rot = (uint32_t)(state >> 59);",
     "    uint64_t old = state;\n    state = state * MUL + INC;\n    uint32_t xorshifted = (uint32_t)(((old >> 18) ^ old) >> 27);\n    uint32_t rot = (uint32_t)(old >> 59);",
     ["test_kat_seed_from_u64_is_pcg32"]),
    # compositions (test_oracle_compositions.py)
    ("PQ generator reseeded per subspace",
     "    size_t w = L.widths[s], off = L.offsets[s];",
     "    seed_from_u64(rng, seed);\n    size_t w = L.widths[s], off = L.offsets[s];",
     ["test_pq_train_one_generator_across_subspaces", "test_pq_twin_subspaces_get_different_codebooks"]),
    ("PQ padding repeats the first centroid",
     "cents.data() + (produced - 1) * w",
     "cents.data()",
     ["test_pq_padding_repeats_the_last_centroid", "test_pq_train_one_generator_across_subspaces"]),
    ("Box-Muller draws swapped",
     "  float u1 = std::fmax(rng.gen_f32(), 1.17549435e-38f);\n  float u2 = rng.gen_f32();",
     "  float u2 = rng.gen_f32();\n  float u1 = std::fmax(rng.gen_f32(), 1.17549435e-38f);",
     ["test_fixture_draw_order_and_box_muller"]),
    ("fixture query noise scale",
     "fixture_gaussian(rng) * 0.25f",
     "fixture_gaussian(rng) * 0.5f",
     ["test_fixture_draw_order_and_box_muller"]),
    ("fixture query source without the stride",
     "    size_t src = (q * stride) % count;",
     "    size_t src = q % count;",
     ["test_fixture_draw_order_and_box_muller"]),
    ("k-means++ cumulative sum in f32",
     "  double cum = 0.0;\n  size_t index = n - 1;",
     "  float cum = 0.0f;\n  size_t index = n - 1;",
     ["test_pp_pick_accumulates_in_f64", "test_kmeans_pp_composition"]),
    ("k-means++ pick with > for >=",
     "    if (cum >= target) {",
     "    if (cum > target) {",
     ["test_pp_pick_first_index_reaching_target"]),
    ("IVF PQ seeded apart from the coarse stage",
     "  pq_train(resid.data(), sampled, dim, m, max_iter, seed, books_out, &rin, &rit);",
     "  pq_train(resid.data(), sampled, dim, m, max_iter, seed + 1, books_out, &rin, &rit);",
     ["test_ivf_train_composition"]),
    ("IVF PQ trained on the sample, not its residuals",
     "  pq_train(resid.data(), sampled, dim, m, max_iter, seed, books_out, &rin, &rit);",
     "  pq_train(sample.data(), sampled, dim, m, max_iter, seed, books_out, &rin, &rit);",
     ["test_ivf_train_composition"]),
    ("IVF stride sample floored",
     "  size_t stride = std::max<size_t>((L + training_sample - 1) / training_sample, 1);",
     "  size_t stride = std::max<size_t>(L / training_sample, 1);",
     ["test_ivf_train_composition"]),
    ("IVF coarse ties by descending list",
     "        return a.second < b.second;",
     "        return a.second > b.second;",
     ["test_ivf_search_composition_l2"]),
    ("IVF shortlist ignores k",
     "      size_t shortlist = rerank > 0 ? std::max(rerank, k) : k;",
     "      size_t shortlist = rerank > 0 ? rerank : k;",
     ["test_ivf_search_composition_l2", "test_ivf_search_composition_cosine_filter_and_untrained_shape"]),
    ("IVF nprobe not clamped below",
     "  size_t np = std::min(std::max<size_t>(nprobe, 1), std::max<size_t>(produced, 1));",
     "  size_t np = std::min(nprobe, produced);",
     ["test_ivf_search_composition_l2"]),
    ("IVF cosine score without the centroid term",
     "arm_nan(1.0f - qdc)",
     "arm_nan(1.0f)",
     ["test_ivf_search_composition_cosine_filter_and_untrained_shape"]),
    ("IVF rerank keeps the ADC score",
     "        exact.push(h.id, space_distance(metric, qv, vectors + s * dim, dim));",
     "        exact.push(h.id, h.d);",
     ["test_ivf_search_composition_l2", "test_ivf_search_composition_cosine_filter_and_untrained_shape"]),
]

_HERE = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_HERE)


def _run_mutant(tmp, i, src, old, new):
    assert src.count(old) == 1, f"mutation site {i} not unique"
    mdir = os.path.join(tmp, f"m{i}")
    os.makedirs(mdir)
    cpp = os.path.join(mdir, "oracle.cpp")
    with open(cpp, "w") as f:
        f.write(src.replace(old, new))
    so = os.path.join(mdir, "liboracle.so")
    subprocess.run(["g++", "-O1", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-pthread",
                    "-shared", "-o", so, cpp], check=True)
    env = dict(os.environ, PXG_ORACLE_LIB=so)
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-rf",
                          os.path.join(_HERE, "test_oracle_pins.py"), os.path.join(_HERE, "test_oracle_compositions.py"),
                          "-k", "not planted"],
                         capture_output=True, text=True, cwd=_ROOT, env=env)
    return set(re.findall(r"FAILED \S*::(\w+)", res.stdout))


def test_planted_mistakes_are_caught():
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    src = open(os.path.join(_ROOT, "oracle", "oracle.cpp")).read()
    with tempfile.TemporaryDirectory() as tmp:
        with ThreadPoolExecutor(4) as pool:
            futs = [pool.submit(_run_mutant, tmp, i, src, old, new) for i, (_, old, new, _) in enumerate(MUTANTS)]
            failed = [f.result() for f in futs]
    for (name, _, _, must), got in zip(MUTANTS, failed):
        missing = set(must) - got
        assert not missing, f"mutant '{name}': these pins still pass: {sorted(missing)} (failed: {sorted(got)})"
