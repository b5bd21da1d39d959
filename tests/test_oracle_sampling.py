"""The sampling oracle against closed forms and frequencies (CPU).

Each check is one a plausible slip would fail: a top-p cut one element off, a cumsum
compared with >= instead of >, an acceptance ratio inverted (q/p), the residual taken as
q - p, or the bonus token drawn from the wrong position."""

import numpy as np
import torch

from oracle.sampling import (chain_speculative_sampling, logits_pipe, sample_from_probs, topk_candidates,
                             verify_topk_speculation)


def chi2_ok(counts, probs, n):
    """Pearson chi-square below the 0.999 quantile for its degrees of freedom (<= 10 cells)."""
    probs = np.asarray(probs, dtype=np.float64)
    keep = probs > 0
    exp = probs[keep] * n
    stat = float((((counts[keep] - exp) ** 2) / exp).sum())
    crit = {1: 10.83, 2: 13.82, 3: 16.27, 4: 18.47, 5: 20.52, 6: 22.46, 7: 24.32, 8: 26.12, 9: 27.88}
    return stat < crit[int(keep.sum()) - 1], stat


def test_topk_candidates_order_ties_and_padding():
    logits = torch.tensor([[1.0, 3.0, 3.0, -2.0, 3.0, 0.5]], dtype=torch.bfloat16)
    v, i = topk_candidates(logits, 4, vocab_start=100)
    assert i.tolist() == [[101, 102, 104, 100]]             # equal 3.0s by id, then the 1.0
    assert v.float().tolist() == [[3.0, 3.0, 3.0, 1.0]]
    v, i = topk_candidates(logits, 8)                        # wider than the shard: -inf / id 0 padding
    assert i[0, 6:].tolist() == [0, 0] and torch.isinf(v[0, 6:].float()).all()
    assert i[0, :6].tolist() == [1, 2, 4, 0, 5, 3]
    # -0 and +0 compare equal: a tie, ordered by id
    z = torch.tensor([[-0.0, 0.0, -1.0]], dtype=torch.bfloat16)
    assert topk_candidates(z, 2)[1].tolist() == [[0, 1]]


def test_logits_pipe_closed_forms():
    x = torch.log(torch.tensor([[0.5, 0.3, 0.2], [0.25, 0.25, 0.5]], dtype=torch.float64)).float()
    p = logits_pipe(x)
    assert torch.allclose(p, torch.tensor([[0.5, 0.3, 0.2], [0.25, 0.25, 0.5]]), atol=1e-6)
    # top_p 0.6: the 0.5 alone misses it, 0.5 + 0.3 reaches it
    assert torch.allclose(logits_pipe(x[:1], top_p=0.6), torch.tensor([[0.625, 0.375, 0.0]]), atol=1e-6)
    # top_p 0.45: the largest alone reaches it
    assert torch.allclose(logits_pipe(x[:1], top_p=0.45), torch.tensor([[1.0, 0.0, 0.0]]), atol=1e-6)
    # a tie at the cut keeps both equal members: 0.5 then the two 0.25s
    assert torch.allclose(logits_pipe(x[1:], top_p=0.6), torch.tensor([[0.25, 0.25, 0.5]]), atol=1e-6)
    # temperature: t = 2 halves the log-probabilities (p^(1/2) normalised); t = 1 is the identity
    p2 = logits_pipe(x[:1], temperature=2.0)
    want = torch.sqrt(torch.tensor([0.5, 0.3, 0.2], dtype=torch.float64))
    assert torch.allclose(p2[0].double(), want / want.sum(), atol=1e-6)
    assert torch.allclose(logits_pipe(x, temperature=1.0), p, atol=1e-7)
    # top_p >= 1 or <= 0: plain softmax
    assert torch.equal(logits_pipe(x, top_p=1.0), p) and torch.equal(logits_pipe(x, top_p=0.0), p)


def test_sample_from_probs_inverse_cdf():
    p = torch.tensor([[0.0, 0.25, 0.0, 0.75], [0.0, 0.0, 1.0, 0.0]])
    u = torch.tensor([0.0, 0.999])
    assert sample_from_probs(p, u).tolist() == [1, 2]        # u = 0: the first positive entry
    # exactly on a boundary: the prefix must exceed u * sum, so 0.25 goes to index 3
    assert sample_from_probs(p[:1], torch.tensor([0.25])).tolist() == [3]
    assert sample_from_probs(p[:1], torch.tensor([0.2499])).tolist() == [1]
    # unnormalised weights scale the target
    assert sample_from_probs(torch.tensor([[2.0, 6.0]]), torch.tensor([0.3])).tolist() == [1]
    rng = np.random.default_rng(0)
    probs = np.array([0.1, 0.2, 0.3, 0.4])
    n = 40000
    draws = sample_from_probs(torch.from_numpy(np.tile(probs, (n, 1))), torch.from_numpy(rng.random(n)))
    ok, stat = chi2_ok(np.bincount(draws.numpy(), minlength=4), probs, n)
    assert ok, stat


def test_chain_closed_forms():
    D, V = 3, 5
    rng = np.random.default_rng(1)
    p = torch.from_numpy(rng.dirichlet(np.ones(V), size=(1, D + 1))).float()
    # identical draft and target distributions: every draft accepted (u q < q for u < 1)
    x = torch.tensor([[1, 4, 2]], dtype=torch.int32)
    u = torch.tensor([[0.99, 0.5, 0.0, 0.3]])
    out, acc, em = chain_speculative_sampling(p[:, :D], x, p, u)
    assert em.tolist() == [3] and acc.tolist() == [3]
    assert out[0, :3].tolist() == [1, 4, 2]
    assert out[0, 3].item() == sample_from_probs(p[:, D], u[:, D]).item()   # bonus from p_D
    # disjoint support at position 0: rejected, the token drawn from p_0 (max(0, p - q) = p there)
    q = torch.zeros(1, D, V)
    q[0, :, 0] = 1.0
    t = torch.zeros(1, D + 1, V)
    t[0, :, 1:] = 0.25
    out, acc, em = chain_speculative_sampling(q, torch.zeros(1, D, dtype=torch.int32), t, u)
    assert em.tolist() == [0] and acc.tolist() == [0]
    assert out[0, 0].item() in (1, 2, 3, 4) and out[0, 1:].tolist() == [-1, -1, -1]
    # acceptance is u q < p, not u p < q: q = 0.8, p = 0.4 at the draft token
    q = torch.zeros(1, 1, 2)
    q[0, 0] = torch.tensor([0.8, 0.2])
    t = torch.zeros(1, 2, 2)
    t[0, 0] = torch.tensor([0.4, 0.6])
    t[0, 1] = torch.tensor([0.5, 0.5])
    x = torch.zeros(1, 1, dtype=torch.int32)
    assert chain_speculative_sampling(q, x, t, torch.tensor([[0.49, 0.0]]))[2].item() == 1    # 0.392 < 0.4
    out, _, em = chain_speculative_sampling(q, x, t, torch.tensor([[0.51, 0.0]]))              # 0.408 > 0.4
    assert em.item() == 0 and out[0, 0].item() == 1          # residual max(0, p - q) = [0, 0.4]


def test_chain_preserves_the_target_distribution():
    """The speculative-sampling guarantee: the first emitted token is distributed as p_0 whatever
    q_0 is (draft token x ~ q_0, accepted with min(1, p/q), else drawn from the residual)."""
    rng = np.random.default_rng(2)
    V, n = 5, 40000
    q0 = np.array([0.5, 0.2, 0.1, 0.1, 0.1])
    p0 = np.array([0.1, 0.1, 0.2, 0.3, 0.3])
    x = rng.choice(V, size=n, p=q0)
    dp = torch.from_numpy(np.tile(q0, (n, 1, 1))).float()
    tp = torch.from_numpy(np.tile(np.stack([p0, p0]), (n, 1, 1))).float()
    out, _, _ = chain_speculative_sampling(dp, torch.from_numpy(x[:, None].astype(np.int32)), tp,
                                           torch.from_numpy(rng.random((n, 2))).float())
    ok, stat = chi2_ok(np.bincount(out[:, 0].numpy(), minlength=V), p0, n)
    assert ok, stat


def test_verify_topk_local_vocabulary():
    """Draft and target candidates that coincide with equal probabilities accept every valid
    draft; a draft token outside the target's candidates is rejected (target mass 0 there) and
    replaced by a target candidate; counts past draft_counts are never emitted."""
    R, D, K = 3, 4, 6
    rng = np.random.default_rng(3)
    ids = torch.from_numpy(np.stack([rng.permutation(1000)[:K] for _ in range(R * (D + 1))]).reshape(R, D + 1, K))
    probs = torch.from_numpy(rng.dirichlet(np.ones(K), size=(R, D + 1))).float()
    draft_probs, draft_ids = probs[:, :D].clone(), ids[:, :D].clone()
    draft_tokens = ids[:, :D, 2].to(torch.int32)                     # each a candidate of the target
    draft_tokens[1, 1] = 5000                                          # not among the target's candidates
    draft_ids[1, 1, 0] = 5000
    counts = torch.tensor([4, 4, 2], dtype=torch.int32)
    u = torch.full((R, D + 1), 0.5)
    out, emitted, _ = verify_topk_speculation(draft_probs, draft_ids, draft_tokens, counts, probs, ids, u)
    assert emitted.tolist() == [4, 1, 2]
    assert out[0, :4].tolist() == draft_tokens[0].tolist() and out[0, 4].item() in ids[0, 4].tolist()
    assert out[1, 0].item() == draft_tokens[1, 0].item()
    assert out[1, 1].item() in ids[1, 1].tolist() and out[1, 2:].tolist() == [-1, -1, -1]
    assert out[2, :2].tolist() == draft_tokens[2, :2].tolist() and out[2, 2].item() in ids[2, 2].tolist()
    assert out[2, 3:].tolist() == [-1, -1]
