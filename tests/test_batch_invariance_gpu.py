"""Batch invariance: one sequence's decode output does not depend on what it
is decoded with (the reference asserts this end to end,
tests/test_engine.py:104-114: a prompt alone and inside a batch give the same
greedy tokens).

Attention: a sequence's summation order depends only on its own length (two
waves per unit up to 8192 tokens, four beyond; partitions of 32768 tokens),
never on the batch, the launch order (the kernel's own longest-first order
or the planner kernel's) or the neighbours' lengths, so the outputs of one
sequence alone and in batches of 1..64 with short or 32k neighbours are
compared bit for bit.  Inputs are uniform random words on
the device (any bits will do for an identity)."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

T, HQ, HKV, D, BS = 4, 14, 2, 64, 16


def _inputs(lens, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    need = [(L + BS - 1) // BS for L in lens]
    nb = sum(need) + 1
    words = lambda *shape: torch.randint(-2 ** 31, 2 ** 31 - 1, shape, generator=g, device=dev,
                                         dtype=torch.int32)
    k, v = words(T, HKV, nb * BS, 2), words(T, HKV, nb * BS, 2)
    q = words(T, len(lens), HQ, 2)
    perm = torch.randperm(nb - 1, generator=g, device=dev).to(torch.int32)
    tables = torch.full((len(lens), max(need)), nb - 1, dtype=torch.int32, device=dev)
    at = 0
    for i, m in enumerate(need):
        tables[i, :m] = perm[at:at + m]
        at += m
    return dict(q=q, k=k, v=v, tables=tables, lens=torch.tensor(lens, dtype=torch.int32, device=dev))


def _attn(inp, rows=None, **env):
    from spikeinfer_amd.kernels import paged_spike_attn_decode

    q, tables, lens = inp["q"], inp["tables"], inp["lens"]
    if rows is not None:
        q, tables, lens = q[:, rows].contiguous(), tables[rows].contiguous(), lens[rows].contiguous()
    out = paged_spike_attn_decode(q, inp["k"], inp["v"], tables, lens, head_dim=D, block_size=BS,
                                  num_q_heads=HQ, num_kv_heads=HKV)
    torch.cuda.synchronize()
    return out


@pytest.fixture
def env(monkeypatch):
    from spikeinfer_amd.kernels.spike_attention import decode_attn_workspace_bytes

    def set_(plan=None):
        decode_attn_workspace_bytes.cache_clear()  # its size depends on the plan
        monkeypatch.delenv("SPIKEINFER_AMD_ATTN_PATH", raising=False)
        if plan is None:
            monkeypatch.delenv("SPIKEINFER_AMD_ATTN_PLAN", raising=False)
        else:
            monkeypatch.setenv("SPIKEINFER_AMD_ATTN_PLAN", plan)
    set_()
    yield set_
    decode_attn_workspace_bytes.cache_clear()


def test_config3_shape_alone_and_in_batches(gpu, env):
    """Config 3 (64 sequences, ctx U[128, 192]): each sequence alone, in the
    batch, and in a batch beside a 20,000-token sequence (which moves the
    launch to the longest-first order): identical bytes."""
    g = torch.Generator().manual_seed(31)
    lens = torch.randint(128, 193, (64,), generator=g).tolist()
    inp = _inputs(lens + [20000], 32, gpu)
    print("batch invariance: config 3 shape", flush=True)
    base = _attn(inp, rows=list(range(64)))
    for i in (0, 17, 63):
        assert torch.equal(_attn(inp, rows=[i])[:, 0], base[:, i]), f"sequence {i} alone"
        mixed = _attn(inp, rows=[i, 64])
        assert torch.equal(mixed[:, 0], base[:, i]), f"sequence {i} beside 20k tokens"
    assert torch.equal(_attn(inp)[:, :64], base), "the batch with the long sequence"


def test_config4_shape_alone_and_in_batches(gpu, env):
    """Config-4 lengths (U[4096, 32768]) on 24 sequences plus one of exactly
    8192 tokens: each alone, in the batch, in a sub-batch, and with the
    launch order from the planner kernel instead of the kernel's own:
    identical bytes."""
    g = torch.Generator().manual_seed(41)
    lens = torch.randint(4096, 32769, (24,), generator=g).tolist() + [8192]
    inp = _inputs(lens, 42, gpu)
    print("batch invariance: config 4 shape", flush=True)
    base = _attn(inp)
    env(plan="workspace")
    assert torch.equal(_attn(inp), base), "planner-kernel order"
    env()
    for i in (0, 5, 23, 24):
        assert torch.equal(_attn(inp, rows=[i])[:, 0], base[:, i]), f"sequence {i} alone"
    sub = [3, 24, 7]
    assert torch.equal(_attn(inp, rows=sub), base[:, sub]), "a sub-batch"


def test_long_context_partitions_alone_and_in_batch(gpu, env):
    """A 40,000-token sequence spans two 32,768-token partitions whatever its
    batch: its output alone equals its output beside short sequences."""
    inp = _inputs([40000, 150, 3000], 52, gpu)
    print("batch invariance: 40k sequence", flush=True)
    base = _attn(inp)
    assert torch.equal(_attn(inp, rows=[0])[:, 0], base[:, 0])
    assert torch.equal(_attn(inp, rows=[1])[:, 0], base[:, 1])


def test_partials_entry_alone_and_in_a_large_batch(gpu, env):
    """The split-context partials entry orders its items only up to 4096 of
    them; past that its 4-wave launch is unplanned and still runs a short
    item as a pair of 2-wave units.  Short sequences of 300..3000 tokens
    (3+ steps, where the 4-wave and 2-wave orders would differ) and a long
    one: their partial sums in a batch of 4,099 items equal theirs alone,
    bit for bit."""
    from spikeinfer_amd.kernels import paged_spike_attn_decode_partials

    lens = [int(x) for x in torch.randint(300, 3000, (4099,), generator=torch.Generator().manual_seed(61))]
    lens[17] = 9000
    inp = _inputs(lens, 62, gpu)

    def parts(rows=None):
        q, tables, ln = inp["q"], inp["tables"], inp["lens"]
        if rows is not None:
            q, tables, ln = q[:, rows].contiguous(), tables[rows].contiguous(), ln[rows].contiguous()
        out = paged_spike_attn_decode_partials(q, inp["k"], inp["v"], tables, ln, head_dim=D, block_size=BS,
                                               num_q_heads=HQ, num_kv_heads=HKV, part_len=16384)
        torch.cuda.synchronize()
        return out

    print("batch invariance: partials entry, 4,099 sequences", flush=True)
    base = parts()
    for i in (0, 17, 2048, 4098):
        alone = parts([i])
        assert torch.equal(alone[0, :, 0], base[0, :, i]), f"sequence {i} (len {lens[i]})"


def _small_model(gpu, seed):
    from spikeinfer_amd.model import SpikingDecoder, SpikingQwenConfig

    cfg = SpikingQwenConfig(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                            num_attention_heads=4, num_key_value_heads=2, head_dim=64)
    return SpikingDecoder(cfg, device=gpu, seed=seed, init_std=0.08)


@pytest.mark.parametrize("sampling", ["greedy", "seeded"])
def test_runner_tokens_alone_and_in_batch(gpu, sampling):
    """The reference's test_batching_does_not_change_results
    (tests/test_engine.py:104-114) on the small spiking model: each prompt
    generated alone, then all together, give identical tokens (greedy, and
    seeded top-k sampling, whose per-request generators draw the same
    uniforms whatever the batch).  Every stage is batch-invariant: prefill
    runs prompt by prompt, the decode GEMMs split K the same way at any row
    count (while the routing below keeps them on this library's kernels:
    T * rows <= small_down_max_rows for the down projection), attention sums
    a sequence's tokens in an order fixed by its own length, norms and the
    sampler work per row."""
    from spikeinfer_amd.runner import DecodeRunner
    from spikeinfer_amd.sampler import SamplingParams
    from spikeinfer_amd.spike_cache import PagedSpikeCache

    m = _small_model(gpu, seed=71)
    g = torch.Generator().manual_seed(72)
    lens = (7, 19, 33, 12, 25)
    prompts = [torch.randint(0, 1024, (L,), generator=g).tolist() for L in lens]
    new = 10

    def params(i):
        if sampling == "greedy":
            return SamplingParams(temperature=0.0)
        return SamplingParams(temperature=0.9, top_k=20, seed=900 + i)

    runner = DecodeRunner(m, PagedSpikeCache(2, m.T, m.Hkv, m.D, 64, 16, device=gpu), batch_size=len(prompts),
                          max_model_len=max(lens) + new + 1, max_new_tokens=16)
    print(f"runner invariance: {sampling}", flush=True)
    alone = [runner.generate([p], [params(i)], new, shuffle_blocks=i)[0] for i, p in enumerate(prompts)]
    together = runner.generate(prompts, [params(i) for i in range(len(prompts))], new, shuffle_blocks=99)
    for i in range(len(prompts)):
        assert torch.equal(together[i], alone[i]), f"prompt {i}: {together[i].tolist()} vs {alone[i].tolist()}"


def test_runner_one_bucket_invariant_through_library_gemm(gpu):
    """Past small_down_max_rows the down projection is the library GEMM, whose
    kernel depends on the row count.  A runner whose only graph bucket is its
    batch size runs every step at that row count (rows past the live ones
    read the pad block), so a prompt alone and in the batch still give the
    same tokens.  Routing forced here: every step's down projection goes to
    the library GEMM."""
    from spikeinfer_amd.runner import DecodeRunner
    from spikeinfer_amd.sampler import SamplingParams
    from spikeinfer_amd.spike_cache import PagedSpikeCache

    m = _small_model(gpu, seed=81)
    m.small_down_max_rows = 0
    g = torch.Generator().manual_seed(82)
    lens = (9, 30, 17, 4)
    prompts = [torch.randint(0, 1024, (L,), generator=g).tolist() for L in lens]
    new = 8
    runner = DecodeRunner(m, PagedSpikeCache(2, m.T, m.Hkv, m.D, 64, 16, device=gpu), batch_size=len(prompts),
                          max_model_len=max(lens) + new + 1, max_new_tokens=16, buckets=())
    assert runner.buckets == (len(prompts),)
    print("runner invariance: one bucket, library down projection", flush=True)
    greedy = SamplingParams(temperature=0.0)
    alone = [runner.generate([p], [greedy], new, shuffle_blocks=i)[0] for i, p in enumerate(prompts)]
    together = runner.generate(prompts, [greedy] * len(prompts), new, shuffle_blocks=99)
    for i in range(len(prompts)):
        assert torch.equal(together[i], alone[i]), f"prompt {i}: {together[i].tolist()} vs {alone[i].tolist()}"


def test_down_projection_routing_switch_is_within_one_ulp(gpu):
    """Where the bucket's row count crosses small_down_max_rows (config-5
    shapes: K = 4864, N = 896), one token's down projection moves from this
    library's long-K kernel (4 rows alone) to the library GEMM (256 rows in
    a batch of 64).  The two may round a sum differently; this bounds that:
    every element of both is within 1 bf16 ulp of the fp64 product, so the
    two differ by at most one rounding step."""
    import torch.nn.functional as F
    from spikeinfer_amd.kernels.decoder_ops import linear_decode, pack_linear

    T, n, K, N = 4, 64, 4864, 896
    g = torch.Generator(device=gpu).manual_seed(91)
    y = torch.randn((T, n, K), generator=g, device=gpu).bfloat16()
    w = (torch.randn((N, K), generator=g, device=gpu) * 0.02).bfloat16()
    batch = F.linear(y, w)  # 256 rows: the library GEMM
    wp = pack_linear(w)
    want = (y.double() @ w.double().t())
    for tok in (0, 17, 63):
        print(f"down projection switch: token {tok}", flush=True)
        alone = linear_decode(y[:, tok:tok + 1].contiguous(), wp, None)  # 4 rows: the long-K kernel
        torch.cuda.synchronize()
        ref = want[:, tok:tok + 1].to(torch.bfloat16).float()
        bound = ref.abs() * 2.0 ** -7 + 1e-6
        assert bool(((alone.float() - ref).abs() <= bound).all())
        assert bool(((batch[:, tok:tok + 1].float() - ref).abs() <= bound).all())
        assert bool(((alone.float() - batch[:, tok:tok + 1].float()).abs() <= 2 * bound).all())
