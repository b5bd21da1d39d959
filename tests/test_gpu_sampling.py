"""Sampling and speculative verification kernels on the GPU against the CPU oracle, with the
same uniforms. Integer outputs must match exactly wherever the decision is not within float
rounding of a boundary (such draws are counted and must be rare); probabilities match within
fp32 rounding. A frequency test checks the GPU chain keeps the target distribution on its own."""

import numpy as np
import pytest
import torch

from aspire_amd.engine.sampling import local_topk_candidates, merge_topk_candidates, verify_topk_speculation
from aspire_amd.logits_processor import build_logits_pipe, define_logit_process_op
from aspire_amd.sampling import chain_speculative_sampling, sampling_from_probs
from helpers import say
from oracle import sampling as osamp

pytestmark = pytest.mark.gpu

MARGIN = 1e-5


@pytest.mark.parametrize("rows,vocab,k,start", [(208, 151936, 50, 0), (33, 1000, 64, 7), (5, 37, 50, 151936),
                                                 (4, 4096, 1024, 0), (2, 155648, 64, 0), (3, 262152, 50, 0),
                                                 (2, 262151, 50, 0)])
def test_topk_candidates_exact(gpu, rows, vocab, k, start):
    """Rows kept in registers (up to 155,648 logits, the largest filling every register slot),
    rows streamed with 16-byte loads (262,152) and with element loads (an odd row length)."""
    say("topk candidates", rows, vocab, k)
    g = torch.Generator().manual_seed(vocab + k)
    # coarse logits: many equal bf16 values, so the tie rule decides the boundary
    logits = (torch.randn(rows, vocab, generator=g) * 3).round().to(torch.bfloat16)
    logits[0, :5] = float("inf")                                  # +inf sorts above every finite logit
    vals, ids = local_topk_candidates(logits.to(gpu), k, vocab_start=start)
    torch.cuda.synchronize()
    ref_v, ref_i = osamp.topk_candidates(logits, k, vocab_start=start)
    assert torch.equal(ids.cpu(), ref_i)
    assert torch.equal(vals.cpu().view(torch.int16), ref_v.view(torch.int16))


@pytest.mark.parametrize("case", ["continuous", "all_equal", "misaligned", "equal_blocks", "outliers", "clustered",
                                  "all_negative"])
def test_topk_candidates_paths(gpu, case):
    """Both collection paths and both load widths: continuous logits (few ties: one pass over every
    key >= the k-th), rows of one repeated value and rows where the boundary value repeats
    thousands of times (ties overflow the candidate buffer: the id-ordered tie ranking), and a
    view whose rows start 2 bytes past a 16-byte boundary (2-byte loads); and rows whose largest
    keys are a few outliers far above the rest, so the boundary lies many bins below the
    maximum's; rows whose largest keys all belong to one thread (ids 8 * 1024 * j + e), so
    its share of the candidates overflows its LDS region and the row takes the full passes; and
    rows of negative logits only (the register slots past a row must stay below every key)."""
    say("topk candidates path", case)
    g = torch.Generator().manual_seed(11)
    rows, vocab, k = 6, 20016, 100
    if case == "continuous":
        logits = torch.randn(rows, vocab, generator=g).to(torch.bfloat16)
    elif case == "all_equal":
        logits = torch.full((rows, vocab), 0.5).to(torch.bfloat16)
        logits[1] = -3.0
    elif case == "misaligned":
        logits = (torch.randn(rows, vocab, generator=g) * 3).round().to(torch.bfloat16)
    elif case == "all_negative":
        logits = (-(torch.randn(rows, vocab, generator=g).abs() + 1.0)).to(torch.bfloat16)
    elif case == "clustered":
        logits = torch.randn(rows, vocab, generator=g)
        ids = torch.tensor([8192 * j + e for j in range((vocab + 8191) // 8192) for e in range(8)
                            if 8192 * j + e < vocab])
        logits[:, ids] = 50.0 + torch.rand(rows, len(ids), generator=g)
        logits = logits.to(torch.bfloat16)
    elif case == "outliers":
        logits = torch.randn(rows, vocab, generator=g)
        logits[:, 100:110] = 1000.0                # 10 keys far above the rest, k = 100
        logits[2, 7] = -1000.0
        logits = logits.to(torch.bfloat16)
    else:
        logits = torch.zeros(rows, vocab).to(torch.bfloat16)
        logits[:, ::7] = 1.0                       # ~2,860 keys tie at the boundary value
        logits[:, 5:40] = 2.0                      # 35 strictly above it
    x = logits.to(gpu) if case != "misaligned" else torch.cat(
        [torch.zeros(rows, 1, dtype=torch.bfloat16), logits], 1).to(gpu)[:, 1:]
    assert (x.data_ptr() % 16 != 0) == (case == "misaligned")
    vals, ids = local_topk_candidates(x, k)
    torch.cuda.synchronize()
    ref_v, ref_i = osamp.topk_candidates(logits, k)
    assert torch.equal(ids.cpu(), ref_i)
    assert torch.equal(vals.cpu().view(torch.int16), ref_v.view(torch.int16))


def test_merge_topk_candidates(gpu):
    g = torch.Generator().manual_seed(3)
    vals = (torch.randn(6, 4 * 50, generator=g) * 2).round().to(torch.bfloat16)
    ids = torch.randint(0, 151936, (6, 200), generator=g)
    mv, mi = merge_topk_candidates(vals.to(gpu), ids.to(gpu), 50)
    rv, ri = osamp.topk_candidates(vals, 50)
    assert torch.equal(mv.cpu().view(torch.int16), rv.view(torch.int16))
    assert torch.equal(mi.cpu(), torch.gather(ids, 1, ri))


@pytest.mark.parametrize("temperature,top_p,dtype", [(0.7, 0.9, torch.bfloat16), (1.0, 0.5, torch.float32),
                                                     (1.3, 0.0, torch.bfloat16), (0.0, 0.95, torch.float32)])
def test_logits_pipe_matches_oracle(gpu, temperature, top_p, dtype):
    say("logits pipe", temperature, top_p, dtype)
    g = torch.Generator().manual_seed(int(temperature * 10 + top_p * 100))
    vals = (torch.randn(64, 50, generator=g) * 2).to(dtype)
    vals[3, 10:] = float("-inf")                                  # a padded narrow shard
    pipe, kw = build_logits_pipe(temperature, top_p)
    probs = pipe(vals.to(gpu), **kw)
    torch.cuda.synchronize()
    ref = osamp.logits_pipe(vals.float(), temperature=temperature if temperature > 0 else None,
                            top_p=top_p if top_p > 0 else None)
    got = probs.cpu()
    skipped = 0
    for r in range(64):
        if top_p > 0:
            base = osamp.logits_pipe(vals[r : r + 1].float(), temperature=temperature if temperature > 0 else None)
            if osamp.cut_margin(base[0].numpy(), top_p) < MARGIN:
                skipped += 1
                continue
            assert torch.equal(got[r] > 0, ref[r] > 0), r                # the same kept set
        assert torch.allclose(got[r], ref[r], rtol=1e-5, atol=1e-7), r
    assert skipped <= 2


def test_sampling_from_probs_matches_oracle(gpu):
    say("sampling_from_probs")
    rng = np.random.default_rng(4)
    R, V = 512, 51
    p = rng.dirichlet(np.full(V, 0.3), size=R).astype(np.float32)
    p[::7, 20:] = 0                                                  # zero tails
    u = rng.random(R).astype(np.float32)
    u[0] = 0.0
    got = sampling_from_probs(torch.from_numpy(p).to(gpu), uniforms=torch.from_numpy(u).to(gpu)).cpu()
    ref = osamp.sample_from_probs(torch.from_numpy(p), torch.from_numpy(u))
    amb = [r for r in range(R) if osamp.draw_margin(p[r], float(u[r])) < MARGIN]
    ok = [r for r in range(R) if r not in amb]
    assert got.dtype == torch.int32 and len(amb) <= 3
    assert torch.equal(got[ok].long(), ref[ok])
    # a wide row (the whole vocabulary) through the chunked scan
    big = rng.random((4, 151936)).astype(np.float32) ** 8
    ub = rng.random(4).astype(np.float32)
    gb = sampling_from_probs(torch.from_numpy(big).to(gpu), uniforms=torch.from_numpy(ub).to(gpu)).cpu()
    rb = osamp.sample_from_probs(torch.from_numpy(big), torch.from_numpy(ub))
    for r in range(4):
        if osamp.draw_margin(big[r], float(ub[r])) >= MARGIN:
            assert gb[r].item() == rb[r].item()


def _chain_inputs(rng, R, D, V, agree=0.6):
    target = rng.dirichlet(np.full(V, 0.5), size=(R, D + 1)).astype(np.float32)
    noise = rng.dirichlet(np.full(V, 0.5), size=(R, D)).astype(np.float32)
    draft = (agree * target[:, :D] + (1 - agree) * noise).astype(np.float32)
    x = np.stack([[rng.choice(V, p=draft[r, i] / draft[r, i].sum()) for i in range(D)] for r in range(R)])
    return draft, x.astype(np.int32), target


def test_chain_speculative_sampling_matches_oracle(gpu):
    say("chain speculative sampling")
    rng = np.random.default_rng(5)
    R, D, V = 256, 5, 51
    draft, x, target = _chain_inputs(rng, R, D, V)
    u = rng.random((R, D + 1)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(gpu)
    acc_in = torch.full((R,), 3, dtype=torch.int32, device=gpu)
    out, acc, em = chain_speculative_sampling(t(draft), t(x), t(target), maybe_output_accepted_token_num=acc_in,
                                              uniforms=t(u))
    torch.cuda.synchronize()
    ref_out, ref_acc, ref_em = osamp.chain_speculative_sampling(torch.from_numpy(draft), torch.from_numpy(x),
                                                                torch.from_numpy(target), torch.from_numpy(u))
    amb = [r for r in range(R) if osamp.chain_draw_margin(torch.from_numpy(draft), torch.from_numpy(x),
                                                          torch.from_numpy(target), torch.from_numpy(u), r) < MARGIN]
    ok = [r for r in range(R) if r not in amb]
    assert len(amb) <= 3
    assert torch.equal(out.cpu()[ok], ref_out[ok])
    assert torch.equal(em.cpu()[ok], ref_em[ok])
    assert torch.equal(acc.cpu()[ok], ref_acc[ok] + 3)            # added in place
    assert acc is acc_in and 0 < int(ref_em.sum()) < R * D         # a mix of accepts and rejects


def test_chain_keeps_the_target_distribution_on_gpu(gpu):
    """Frequency check of the GPU kernel alone: the first emitted token follows p_0 for any q_0."""
    say("chain frequency")
    rng = np.random.default_rng(6)
    V, n = 6, 200000
    q0 = np.array([0.4, 0.3, 0.1, 0.1, 0.05, 0.05])
    p0 = np.array([0.05, 0.1, 0.15, 0.2, 0.2, 0.3])
    x = torch.from_numpy(rng.choice(V, size=(n, 1), p=q0).astype(np.int32)).to(gpu)
    dp = torch.from_numpy(q0.astype(np.float32)).to(gpu).expand(n, 1, V).contiguous()
    tp = torch.from_numpy(np.stack([p0, p0]).astype(np.float32)).to(gpu).expand(n, 2, V).contiguous()
    out, _, _ = chain_speculative_sampling(dp, x, tp, generator=torch.Generator(device=gpu).manual_seed(1))
    counts = np.bincount(out[:, 0].cpu().numpy(), minlength=V)
    exp = p0 * n
    stat = float(((counts - exp) ** 2 / exp).sum())
    assert stat < 20.52, stat                                      # chi-square 0.999 quantile, 5 dof


@pytest.mark.parametrize("R,K", [(64, 50), (16, 1024)])
def test_verify_topk_speculation_matches_oracle(gpu, R, K):
    """Small candidate lists and the largest top_k (1,024: the draft probabilities map onto the
    target's candidates through the kernel's sorted id table), with a repeated draft id in one
    row (its probabilities add up, as the reference's masked sum does)."""
    say("verify_topk_speculation", R, K)
    rng = np.random.default_rng(7 + K)
    D, vocab = 6, 151936
    target_ids = np.stack([rng.choice(vocab, size=K, replace=False) for _ in range(R * (D + 1))]).reshape(R, D + 1, K)
    # draft candidates: mostly the target's, some replaced by other ids, in another order
    draft_ids = target_ids[:, :D].copy()
    for r in range(R):
        for i in range(D):
            draft_ids[r, i] = rng.permutation(draft_ids[r, i])
            swap = rng.random(K) < 0.2
            draft_ids[r, i, swap] = rng.choice(vocab, size=int(swap.sum()), replace=False) + vocab
    draft_ids[0, 0, 1] = draft_ids[0, 0, 0]
    target_probs = rng.dirichlet(np.full(K, 0.4), size=(R, D + 1)).astype(np.float32)
    draft_probs = rng.dirichlet(np.full(K, 0.4), size=(R, D)).astype(np.float32)
    tok = np.stack([[draft_ids[r, i, rng.choice(K, p=draft_probs[r, i])] for i in range(D)] for r in range(R)])
    counts = rng.integers(0, D + 1, size=R).astype(np.int32)
    u = rng.random((R, D + 1)).astype(np.float32)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    out, emitted = verify_topk_speculation(T(draft_probs).to(gpu), T(draft_ids).to(gpu), T(tok.astype(np.int32)).to(gpu),
                                           T(counts).to(gpu), T(target_probs).to(gpu), T(target_ids).to(gpu),
                                           uniforms=T(u).to(gpu))
    torch.cuda.synchronize()
    ref_out, ref_em, (ld, lt, ltg) = osamp.verify_topk_speculation(T(draft_probs), T(draft_ids), T(tok.astype(np.int32)),
                                                                   T(counts), T(target_probs), T(target_ids), T(u))
    amb = [r for r in range(R) if osamp.chain_draw_margin(ld, lt, ltg, T(u), r) < MARGIN]
    ok = [r for r in range(R) if r not in amb]
    assert len(amb) <= 2
    assert out.dtype == torch.int64 and emitted.dtype == torch.int32
    assert torch.equal(out.cpu()[ok], ref_out[ok])
    assert torch.equal(emitted.cpu()[ok], ref_em[ok])
    assert 0 < int(ref_em.sum()) < int(counts.sum())


def _f32_chunk_prefixes(w: np.ndarray, threads: int = 256):
    """The draw's fp32 chunk partition: chunk length, per-chunk sums (from 0, in index order) and
    the exclusive prefixes of those sums in thread order, as the scan adds them."""
    chunk = -(-w.size // threads)
    part = np.zeros(threads, dtype=np.float32)
    for t in range(threads):
        acc = np.float32(0)
        for x in w[t * chunk : (t + 1) * chunk]:
            acc = np.float32(acc + x)
        part[t] = acc
    excl = np.zeros(threads + 1, dtype=np.float32)
    for t in range(threads):
        excl[t + 1] = np.float32(excl[t] + part[t])
    return chunk, part, excl


def test_draw_at_chunk_boundaries_never_takes_a_zero_weight(gpu):
    """Inverse-CDF draws over 4,096 weights (chunks of 16 per thread) whose target sits just below
    each chunk boundary's prefix, with the next chunk starting on a weight of 0: the drawn index
    lies in the chunk that ends at the boundary and never has weight 0 (a draw that summed the
    chunk in another order than its check could hit the next chunk's zero)."""
    say("draw chunk boundaries")
    rng = np.random.default_rng(8)
    n = 4096
    w = (rng.random(n) * 0.9 + 0.1).astype(np.float32) / np.float32(7.3)
    chunk, part, excl = _f32_chunk_prefixes(w)
    w[chunk::chunk] = 0
    chunk, part, excl = _f32_chunk_prefixes(w)
    total = excl[-1]
    us, bounds = [], []
    for c in range(1, n // chunk):
        target = np.nextafter(excl[c], np.float32(0))             # just below the boundary prefix
        u = np.float32(target / total)
        while np.float32(u * total) >= excl[c]:
            u = np.nextafter(u, np.float32(0))
        while np.float32(np.nextafter(u, np.float32(1)) * total) < excl[c]:
            u = np.nextafter(u, np.float32(1))
        us.append(u)
        bounds.append(c)
    R = len(us)
    probs = torch.from_numpy(np.tile(w, (R, 1))).to(gpu)
    got = sampling_from_probs(probs, uniforms=torch.from_numpy(np.array(us, dtype=np.float32)).to(gpu)).cpu().numpy()
    for r, c in enumerate(bounds):
        assert w[got[r]] > 0, (c, got[r])
        assert (c - 1) * chunk <= got[r] < c * chunk, (c, got[r])


def test_top_p_cut_at_chunk_boundaries(gpu):
    """Top-p over 4,096 candidates (sorted prefix sums in chunks of 16 per thread) with top_p
    equal to the fp32 prefix at a chunk boundary: exactly one thread finds the cut, inside the
    chunk that ends there, so the kept set is that chunk's prefix (not every candidate, and not a
    cut past the boundary)."""
    say("top-p chunk boundaries")
    g = torch.Generator().manual_seed(9)
    # distinct logits 0.002 apart: every probability differs from the next by a factor 1.002
    vals = (torch.randperm(4096, generator=g).float() * 0.002).view(1, 4096).to(gpu)
    pipe, _ = build_logits_pipe(0.0, 0.0)
    probs = pipe(vals).cpu().numpy()[0]                            # the kernel's own probabilities
    srt = np.sort(probs)[::-1].astype(np.float32)
    assert np.unique(srt).size == srt.size
    chunk, part, excl = _f32_chunk_prefixes(srt)
    top_pipe, _ = build_logits_pipe(0.0, 0.5)
    for c in (3, 17, 64, 100, 128, 181, 250):
        top_p = float(excl[c])
        if not 0.0 < top_p < 1.0 or not excl[c - 1] < excl[c]:
            continue
        kept = int((top_pipe(vals, top_p=top_p).cpu().numpy()[0] > 0).sum())
        assert (c - 1) * chunk < kept <= c * chunk, (c, kept)


def test_sampling_graph_replays(gpu):
    """Top-k + pipe + draws captured in a HIP graph with torch.rand uniforms: each replay draws
    new uniforms, and each replay's tokens equal the oracle's on that replay's uniforms."""
    say("sampling graph")
    g = torch.Generator().manual_seed(9)
    logits = torch.randn(16, 8192, generator=g).to(torch.bfloat16).to(gpu)
    pipe, kw = build_logits_pipe(0.8, 0.9)
    u = torch.empty(16, device=gpu)
    out = torch.empty(16, dtype=torch.int32, device=gpu)
    probs_buf = torch.empty(16, 50, device=gpu)

    def step():
        vals, ids = local_topk_candidates(logits, 50)
        probs_buf.copy_(pipe(vals, **kw))
        u.copy_(torch.rand(16, device=gpu))
        out.copy_(sampling_from_probs(probs_buf, uniforms=u))

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    seen = []
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        ref = osamp.sample_from_probs(probs_buf.cpu(), u.cpu())
        for r in range(16):
            if osamp.draw_margin(probs_buf[r].cpu().numpy(), float(u[r])) >= MARGIN:
                assert out[r].item() == ref[r].item(), (rep, r)
        seen.append(u.cpu().clone())
        _ = torch.randn(100, device=gpu).sum().item()
    assert not torch.equal(seen[0], seen[1])


def test_logit_process_op(gpu):
    pipe, kw = build_logits_pipe(0.9, 0.8)
    op = define_logit_process_op(pipe, kw)
    vals = torch.randn(8, 50, device=gpu).to(torch.bfloat16)
    assert torch.equal(op(vals), pipe(vals, **kw))
    with torch._subclasses.fake_tensor.FakeTensorMode():
        fake = torch.empty(8, 50, dtype=torch.bfloat16, device=gpu)
        assert op(fake).dtype == torch.float32
