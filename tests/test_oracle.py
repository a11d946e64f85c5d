"""Pins the CPU oracle before anything is checked against it (CPU only).

Each check is chosen so a plausible mistake in the restatement fails it: the
reference's own known-answer tests, closed forms, independent formulations
(numpy.packbits, numpy float32 stepping, pure-Python attention) and
invariants the reference tests assert.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from cases import attn_case, oracle_attn, random_bits
from oracle import oracle as orc


# ---- packing: tests/test_packing.py known answers -------------------------
@pytest.mark.parametrize("channels", [1, 31, 32, 33, 63, 64, 128, 256, 4864])
def test_pack_matches_packbits_and_roundtrips(channels):
    rng = np.random.default_rng(channels)
    bits = random_bits(rng, (3, 5, channels), 0.5)
    words = orc.pack(bits)
    assert words.dtype == np.int32 and words.shape == (3, 5, (channels + 31) // 32)
    assert np.array_equal(words, orc.np_pack(bits))
    assert np.array_equal(orc.unpack(words, channels), bits)
    assert np.array_equal(orc.np_unpack(words, channels), bits)


def test_all_ones_is_minus_one():
    # tests/test_packing.py:45-50
    assert orc.pack(np.ones((1, 32), np.uint8)).item() == -1


@pytest.mark.parametrize("channel", [0, 1, 31, 32, 63])
def test_bit_order_little_endian(channel):
    # tests/test_packing.py:53-63: channel c -> bit c % 32 of word c // 32
    bits = np.zeros((1, 64), np.uint8)
    bits[0, channel] = 1
    w = orc.pack(bits)[0].view(np.uint32)
    want = [0, 0]
    want[channel // 32] = 1 << (channel % 32)
    assert w.tolist() == want
    # ...and the two words are the little-endian uint64 with bit c set.
    assert orc.pack(bits)[0].view("<u8").item() == 1 << channel


def test_tail_word_of_c33():
    # tests/test_packing.py:66-70
    assert orc.pack(np.ones((1, 33), np.uint8))[0, 1] == 1


def test_graded_values_count_as_spikes():
    # tests/test_packing.py:73-80
    words = orc.pack(np.array([[0.0, 0.5, 0.0, 2.0]]))
    assert orc.unpack(words, 4).tolist() == [[0, 1, 0, 1]]


def test_packed_bytes_per_token_known_answer():
    # tests/test_packing.py:89-99 and README.md:59-62
    from spikeinfer_amd.kernels.packing import packed_bytes_per_token, packed_width

    assert packed_bytes_per_token(24, 4, 2, 64) == 3072
    assert [packed_width(c) for c in (1, 31, 32, 33, 64, 4864)] == [1, 1, 1, 2, 2, 152]


# ---- LIF: lif_triton.py recurrence ----------------------------------------
def test_lif_hand_case():
    # beta=0.9, theta=1, I=1: u = 1.0 sits exactly on theta at t=0 (no spike);
    # then 1.9 (spike), 0.9*1.9+1-1 = 1.71 (spike), 1.539 (spike).
    x = np.ones((4, 1, 1), np.float32)
    spk, u = orc.lif(x, np.array([0.9], np.float32), np.array([1.0], np.float32))
    assert spk[:, 0, 0].tolist() == [0, 1, 1, 1]
    b = np.float32(0.9)
    want = np.float32(1.0)
    for _ in range(3):
        want = (b * want + np.float32(1)) - (np.float32(1) if want - 1 > 0 else np.float32(0))
    assert u[0, 0] == want


@pytest.mark.parametrize("T", [1, 2, 4, 8])
@pytest.mark.parametrize("N", [64, 63, 4864])
def test_lif_c_matches_numpy_float32(T, N):
    rng = np.random.default_rng(1000 * T + N)
    beta = (rng.random(N) * 4 - 1.5).astype(np.float32)  # exercises the clamp
    thr = (rng.random(N) * 0.95 + 0.05).astype(np.float32)
    x = (rng.standard_normal((T, 37, N)) * 2).astype(np.float32)
    s1, u1 = orc.lif(x, beta, thr)
    s2, u2 = orc.np_lif(x, beta, thr)
    assert np.array_equal(s1, s2)
    assert np.array_equal(u1.view(np.uint32), u2.view(np.uint32))


def test_lif_beta_clamp():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 8, 3)).astype(np.float32)
    thr = np.full(3, 0.5, np.float32)
    a = orc.lif(x, np.array([2.5, -1.0, 0.5], np.float32), thr)
    b = orc.lif(x, np.array([1.0, 0.0, 0.5], np.float32), thr)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_lif_boundary_stress_detects_fma():
    """tests/test_lif_kernel.py:192-210 scenario.  The oracle must agree with
    numpy's two-rounding arithmetic AND differ from a single-rounding (fused)
    evaluation somewhere, or the case would not guard against contraction."""
    rng = np.random.default_rng(0)
    T, M, N = 8, 256, 64
    beta = np.full(N, 0.9, np.float32)
    thr = np.full(N, 1.0, np.float32)
    x = (np.ones((T, M, N)) + rng.standard_normal((T, M, N)) * 1e-6).astype(np.float32)
    s1, u1 = orc.lif(x, beta, thr)
    s2, u2 = orc.np_lif(x, beta, thr)
    assert np.array_equal(s1, s2) and np.array_equal(u1, u2)
    # fused: beta*u + x rounded once (float64 product+sum, then to float32)
    u = np.zeros((M, N), np.float32)
    fused_u = []
    for t in range(T):
        r = ((u - thr) > 0).astype(np.float32)
        u = (beta.astype(np.float64) * u + x[t]).astype(np.float32) - r * thr
        fused_u.append(u)
    assert not np.array_equal(fused_u[-1], u1), "case no longer separates fused from unfused"


def test_lif_mem0():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((3, 4, 5)).astype(np.float32)
    m0 = rng.standard_normal((4, 5)).astype(np.float32)
    b = np.full(5, 0.7, np.float32)
    th = np.full(5, 0.3, np.float32)
    s1, u1 = orc.lif(x, b, th, m0)
    s2, u2 = orc.np_lif(x, b, th, m0)
    assert np.array_equal(s1, s2) and np.array_equal(u1, u2)


def test_lif_pack_write_is_the_composition():
    rng = np.random.default_rng(3)
    T, n_tok, H, D = 4, 6, 2, 64
    x = rng.standard_normal((T, n_tok, H, D)).astype(np.float32)
    b = np.full(D, 0.9, np.float32)
    th = np.full(D, 1.0, np.float32) * 0.5
    buf = np.zeros((T, n_tok, H, 2), np.int32)
    orc.lif_pack_write(x, b, th, buf)
    spk, _ = orc.np_lif(x, b, th)
    assert np.array_equal(buf, orc.np_pack(spk))
    S = 64
    slots = np.array([5, 17, -1, 40, 63, 64], np.int64)
    cache = np.full((T, H, S, 2), 7, np.int32)
    orc.lif_pack_write(x, b, th, cache, slots)
    want = np.full((T, H, S, 2), 7, np.int32)
    for i, s in enumerate(slots):
        if 0 <= s < S:
            want[:, :, s] = orc.np_pack(spk)[:, i]
    assert np.array_equal(cache, want)


# ---- attention -------------------------------------------------------------
@pytest.mark.parametrize("lens,bs", [([1], 4), ([7], 4), ([9, 3, 17], 4), ([5, 16], 8)])
@pytest.mark.parametrize("heads", [(4, 2), (2, 2), (6, 1)])
def test_attention_matches_pure_python(lens, bs, heads):
    case = attn_case(lens, block_size=bs, T=2, q_heads=heads[0], kv_heads=heads[1],
                     head_dim=32 if heads[1] == 1 else 64, seed=len(lens) + bs)
    want = orc.brute_attn(case["q"], case["k"], case["v"], case["tables"], case["lens"],
                          case["head_dim"], bs, *heads)
    got = oracle_attn(case)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_scores_equal_unpacked_dot_products():
    # tests/test_cpu_backend.py:165-181: popcount(q & k) == q . k on bits
    case = attn_case([21, 9], block_size=4, T=2, q_heads=4, kv_heads=2, seed=2)
    sc = orc.decode_scores(case["q"], case["k"], case["tables"], case["lens"], 64, 4, 4, 2, 21)
    qb, kb = orc.np_unpack(case["q"], 64), orc.np_unpack(case["k"], 64)
    for t in range(2):
        for n, L in enumerate(case["lens"]):
            for h in range(4):
                for p in range(21):
                    if p >= L:
                        assert sc[t, n, h, p] == -1
                        continue
                    slot = case["tables"][n, p // 4] * 4 + p % 4
                    assert sc[t, n, h, p] == int(qb[t, n, h].astype(int) @ kb[t, h // 2, slot])


def test_slot_walk_known_answer():
    # tests/test_cpu_backend.py:184-190 (tables [[3,1,7],[5,2,0]], bs=4, len=10):
    # give slot s exactly (s % 33) set bits and an all-ones query, so each
    # score reads back the slot it came from.
    tables = np.array([[3, 1, 7], [5, 2, 0]], np.int32)
    S = 32
    bits = np.zeros((1, 1, S, 64), np.uint8)
    for s in range(S):
        bits[0, 0, s, : s % 33] = 1
    k = orc.pack(bits)
    q = orc.pack(np.ones((1, 2, 1, 64), np.uint8))
    sc = orc.decode_scores(q, k, tables, np.array([10, 10], np.int32), 64, 4, 1, 1, 10)
    assert sc[0, :, 0].tolist() == [[12, 13, 14, 15, 4, 5, 6, 7, 28, 29],
                                    [20, 21, 22, 23, 8, 9, 10, 11, 0, 1]]


def test_zero_query_gives_mean_of_values():
    # tests/test_spike_attention.py:115-134: uniform softmax -> mean of V bits
    case = attn_case([40, 17], block_size=16, T=2, seed=4)
    case["q"][:] = 0
    got = oracle_attn(case)
    vb = orc.np_unpack(case["v"], 64)
    for n, L in enumerate(case["lens"]):
        slots = [case["tables"][n, p // 16] * 16 + p % 16 for p in range(L)]
        for h in range(14):
            np.testing.assert_allclose(got[:, n, h], vb[:, h // 7, slots].mean(axis=1), atol=1e-15)


def test_single_token_returns_its_value_bits():
    case = attn_case([1, 1], block_size=16, seed=6)
    got = oracle_attn(case)
    vb = orc.np_unpack(case["v"], 64)
    for n in range(2):
        slot = case["tables"][n, 0] * 16
        for h in range(14):
            assert np.array_equal(got[:, n, h], vb[:, h // 7, slot].astype(float))


def test_only_own_blocks_and_not_past_len():
    case = attn_case([9, 25, 41, 3], block_size=16, seed=7)
    before = oracle_attn(case)
    owned = set()
    for n, L in enumerate(case["lens"]):
        need = (L + 15) // 16
        owned.update(case["tables"][n, :need].tolist())
        last = case["tables"][n, (L - 1) // 16]
        if L % 16:  # tail of the last block, past seq_len
            case["k"][:, :, last * 16 + L % 16:(last + 1) * 16] = -1
            case["v"][:, :, last * 16 + L % 16:(last + 1) * 16] = -1
    for b in range(case["k"].shape[2] // 16):
        if b not in owned:
            case["k"][:, :, b * 16:(b + 1) * 16] = -1
            case["v"][:, :, b * 16:(b + 1) * 16] = -1
    assert np.array_equal(oracle_attn(case), before)


def test_softmax_is_shift_invariant_closed_form():
    """Two keys with counts c1, c2: weight ratio exp((c1 - c2)/8) exactly."""
    kbits = np.zeros((1, 1, 2, 64), np.uint8)
    kbits[0, 0, 0, :10] = 1
    kbits[0, 0, 1, :3] = 1
    vbits = np.zeros((1, 1, 2, 64), np.uint8)
    vbits[0, 0, 0, 0] = 1
    vbits[0, 0, 1, 1] = 1
    q = orc.pack(np.ones((1, 1, 1, 64), np.uint8))
    out = orc.decode_attn(q, orc.pack(kbits), orc.pack(vbits), np.array([[0]], np.int32),
                          np.array([2], np.int32), 64, 2, 1, 1)
    w0 = 1 / (1 + math.exp(-7 / 8))
    np.testing.assert_allclose(out[0, 0, 0, :2], [w0, 1 - w0], rtol=1e-14)
    assert np.all(out[0, 0, 0, 2:] == 0)


# ---- prefill chunk oracle --------------------------------------------------
def _prefill_case(ctx, q_len, seed=3, T=2, Hq=4, Hkv=2, D=64, bs=4):
    c = attn_case([ctx + q_len], block_size=bs, T=T, q_heads=Hq, kv_heads=Hkv,
                  head_dim=D, seed=seed)
    rng = np.random.default_rng(seed + 100)
    q_bits = random_bits(rng, (T, Hq, q_len, D), 0.4)
    return c, q_bits


@pytest.mark.parametrize("ctx,q_len", [(0, 1), (0, 7), (5, 3), (13, 6)])
def test_prefill_rows_equal_decode_at_their_length(ctx, q_len):
    """Row i of a chunk sees exactly positions [0, ctx + i], so it must equal an
    independent decode (C oracle) with seq_len = ctx + i + 1."""
    c, q_bits = _prefill_case(ctx, q_len)
    got = orc.prefill_attn(q_bits, c["k"], c["v"], c["tables"][0], ctx, 64, 4, 4, 2)
    for i in range(q_len):
        q = orc.np_pack(q_bits[:, :, i][:, None])  # [T, 1, Hq, W]
        want = orc.decode_attn(q, c["k"], c["v"], c["tables"], np.array([ctx + i + 1], np.int32),
                               64, 4, 4, 2)
        np.testing.assert_allclose(got[:, :, i], want[:, 0], rtol=0, atol=1e-12)


def test_prefill_zero_query_is_running_mean():
    c, q_bits = _prefill_case(4, 5)
    q_bits[:] = 0
    got = orc.prefill_attn(q_bits, c["k"], c["v"], c["tables"][0], 4, 64, 4, 4, 2)
    pos = np.arange(9)
    slots = c["tables"][0][pos // 4] * 4 + pos % 4
    vb = orc.np_unpack(c["v"][:, :, slots], 64).astype(np.float64)  # [T, Hkv, 9, D]
    for i in range(5):
        want = vb[:, :, : 4 + i + 1].mean(axis=2)  # [T, Hkv, D]
        np.testing.assert_allclose(got[:, :, i], np.repeat(want, 2, axis=1), atol=1e-12)


# ---- sampler oracle (spikeinfer/engine/sampler.py semantics) ----------------
def test_sample_closed_form_distribution():
    """logits ln(1..4): probabilities k/10, drawn largest first, so the draw's
    boundaries are at .4, .7, .9."""
    lg = np.log(np.arange(1, 5, dtype=np.float64)).astype(np.float32)
    _, kept, probs, _, order = orc.sample_row(lg)
    assert kept.all() and order.tolist() == [3, 2, 1, 0]
    np.testing.assert_allclose(probs, [0.1, 0.2, 0.3, 0.4], atol=1e-7)
    toks = [orc.sample_row(lg, u=u)[0] for u in (0.05, 0.39, 0.41, 0.69, 0.71, 0.89, 0.91, 0.99)]
    assert toks == [3, 3, 2, 2, 1, 1, 0, 0]


def test_sample_top_k_top_p_min_p_known_answers():
    lg = np.log(np.array([1, 2, 3, 4], np.float64)).astype(np.float32)
    assert orc.sample_row(lg, top_k=2)[1].tolist() == [False, False, True, True]
    # top_p 0.5: mass before 0.4 is 0 and before 0.3 is 0.4 (< 0.5): keep {3, 2}
    assert orc.sample_row(lg, top_p=0.5)[1].tolist() == [False, False, True, True]
    # top_p 0.35: the second token has 0.4 before it, not < 0.35: keep {3}
    assert orc.sample_row(lg, top_p=0.35)[1].tolist() == [False, False, False, True]
    # min_p 0.45: keep p >= 0.45 * 0.4 = 0.18
    assert orc.sample_row(lg, min_p=0.45)[1].tolist() == [False, True, True, True]
    assert orc.sample_row(lg, top_k=1)[0] == 3
    assert orc.sample_row(lg, temperature=0.0)[0] == 3


def test_sample_penalties_known_answers():
    lg = np.array([2.0, -2.0, 1.0, 0.5], np.float32)
    # repetition 2 on tokens 0 and 1: 2 -> 1, -2 -> -4; greedy picks token 0 vs 2 (1.0 tie: lowest index)
    assert orc.sample_row(lg, temperature=0.0, rep=2.0, history=[0, 1])[0] == 0
    assert orc.sample_row(lg, temperature=0.0, rep=4.0, history=[0])[0] == 2
    # frequency 0.5 x 3 occurrences + presence 0.25 on token 0: 2 - 1.75 = 0.25 < 0.5
    assert orc.sample_row(lg, temperature=0.0, presence=0.25, frequency=0.5, history=[0, 0, 0])[0] == 2


def test_sample_ties_ordered_by_index():
    lg = np.array([1.0, 3.0, 3.0, 3.0, 0.0], np.float32)
    assert orc.sample_row(lg, top_k=2)[1].tolist() == [False, True, True, False, False]
    assert orc.sample_row(lg, temperature=0.0)[0] == 1
