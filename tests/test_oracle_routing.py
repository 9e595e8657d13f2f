"""Pins the routing oracle (oracle/routing.py): against the reference's own
torch op sequences (model/moe.py:249-281, :1565-1567, :1594) and brute-force
Python loops on small inputs."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import routing as orouting
from tests.helpers import zipf_routing


def test_softmax_topk_matches_reference_ops():
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(2, 300, 8, generator=g)
    vals, idx = logits.topk(2, dim=-1)            # model/moe.py:253
    w = F.softmax(vals, dim=-1)                   # model/moe.py:254
    ow, oidx = orouting.softmax_topk(logits.reshape(-1, 8).numpy(), 2)
    assert np.array_equal(oidx, idx.reshape(-1, 2).numpy())
    assert np.allclose(ow, w.reshape(-1, 2).numpy(), rtol=1e-6, atol=1e-7)
    w1, _ = orouting.softmax_topk(logits.reshape(-1, 8).numpy(), 1)
    assert np.all(w1 == 1.0)


def test_sigmoid_topk_matches_reference_ops():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(500, 64, generator=g) * 3
    s = torch.sigmoid(logits)                     # model/moe.py:260
    vals, idx = s.topk(6, dim=-1)                 # model/moe.py:261
    w = vals / (vals.sum(dim=-1, keepdim=True) + 1e-8)  # model/moe.py:263
    ow, oidx = orouting.sigmoid_topk(logits.numpy(), 6)
    assert np.array_equal(oidx, idx.numpy())
    assert np.allclose(ow, w.numpy(), rtol=1e-6, atol=1e-7)


def test_load_balancing_loss_matches_reference_ops():
    g = torch.Generator().manual_seed(2)
    E, K = 8, 2
    logits = torch.randn(2, 256, E, generator=g)
    _, idx = logits.topk(K, dim=-1)
    # model/moe.py:274-281
    num_tokens = logits.shape[0] * logits.shape[1]
    expert_mask = F.one_hot(idx, E).sum(dim=2)
    f = expert_mask.float().sum(dim=[0, 1]) / num_tokens
    P = F.softmax(logits, dim=-1).float().mean(dim=[0, 1])
    ref = float(E * (f * P).sum())
    got = orouting.load_balancing_loss(logits.numpy(), idx.numpy(), E)
    assert abs(got - ref) < 1e-6


def _brute_force_sort(idx, E, pad=128):
    T, K = idx.shape
    counts = [0] * E
    rows = {}
    off = 0
    offsets = []
    for e in range(E):
        offsets.append(off)
        r = off
        for t in range(T):
            for k in range(K):
                if idx[t, k] == e:
                    rows[t * K + k] = r
                    r += 1
                    counts[e] += 1
        off += -(-counts[e] // pad) * pad
    offsets.append(off)
    return counts, offsets, [rows.get(a, -1) for a in range(T * K)]


@pytest.mark.parametrize("T,E,K,s,zeros", [(300, 4, 1, 0.0, ()), (257, 8, 2, 1.1, (3,)),
                                           (100, 32, 8, 1.2, (0, 1, 31)), (1, 1, 1, 0.0, ())])
def test_sort_matches_brute_force(T, E, K, s, zeros):
    _, idx = zipf_routing(T, E, K, s, seed=T, zero_experts=zeros)
    idx = idx.numpy()
    r = orouting.sort_assignments(idx, E)
    counts, offsets, rows = _brute_force_sort(idx, E)
    assert r["counts"].tolist() == counts
    assert r["offsets"].tolist() == offsets
    assert r["row_of"].tolist() == rows
    aor = r["assign_of_row"]
    assert sorted(aor[aor >= 0].tolist()) == list(range(T * K))
    assert (aor[np.asarray(rows)] == np.arange(T * K)).all()


def test_sort_drops_out_of_range_like_the_reference_loop():
    """Slots routed outside [0, E) (another GPU's experts; negative after an
    expert offset) take no row, as the reference loop walks only the local
    experts (model/moe.py:1560-1567): the kept slots sort exactly as the brute
    force over the in-range slots, and unpermute adds nothing for the others."""
    rng = np.random.default_rng(11)
    T, E, K, D = 120, 6, 4, 8
    idx = rng.integers(-3, E + 5, size=(T, K))
    r = orouting.sort_assignments(idx, E, drop_out_of_range=True)
    counts, offsets, rows = _brute_force_sort(idx, E)   # ignores indices outside [0, E)
    assert r["counts"].tolist() == counts
    assert r["offsets"].tolist() == offsets
    valid = ((idx >= 0) & (idx < E)).reshape(-1)
    assert (r["row_of"][~valid] == -1).all()
    assert np.array_equal(r["row_of"][valid], np.asarray(rows)[valid])
    y = rng.standard_normal((r["assign_of_row"].size, D)).astype(np.float32)
    w = rng.random((T, K)).astype(np.float32)
    out = orouting.unpermute_unpad(y, r["row_of"], w, T, K)
    for t in range(T):
        acc = np.zeros(D, np.float32)
        for k in range(K):
            if 0 <= idx[t, k] < E:
                acc = (acc + w[t, k] * y[r["row_of"][t * K + k]]).astype(np.float32)
        assert np.array_equal(out[t], acc)
    with pytest.raises(ValueError):
        orouting.sort_assignments(idx, E)


def test_sort_order_equals_reference_nonzero():
    """model/moe.py:1566-1567: the tokens of expert e, ascending."""
    _, idx = zipf_routing(500, 8, 2, 0.5, seed=3)
    r = orouting.sort_assignments(idx.numpy(), 8)
    for e in range(8):
        ref = (idx == e).any(dim=-1).nonzero(as_tuple=True)[0].numpy()
        a = r["assign_of_row"][r["offsets"][e]: r["offsets"][e] + r["counts"][e]]
        assert np.array_equal(a // 2, ref)


def test_sort_duplicate_expert_in_one_token():
    idx = np.array([[1, 1], [0, 1]])
    r = orouting.sort_assignments(idx, 2)
    assert r["counts"].tolist() == [1, 3]
    assert r["row_of"].tolist() == [128, 129, 0, 130]


def test_permute_and_unpermute_brute_force():
    rng = np.random.default_rng(0)
    T, E, K, D = 50, 4, 2, 16
    w, idx = zipf_routing(T, E, K, 0.0, seed=5)
    r = orouting.sort_assignments(idx.numpy(), E)
    x = rng.standard_normal((T, D)).astype(np.float32)
    p = orouting.permute_pad(x, r["assign_of_row"], K)
    for row, a in enumerate(r["assign_of_row"]):
        assert np.array_equal(p[row], x[a // K] if a >= 0 else np.zeros(D, np.float32))
    y = rng.standard_normal((p.shape[0], D)).astype(np.float32)
    out = orouting.unpermute_unpad(y, r["row_of"], w.numpy(), T, K)
    for t in range(T):
        acc = np.zeros(D, np.float32)
        for k in range(K):
            acc = (acc + np.float32(w[t, k]) * y[r["row_of"][t * K + k]]).astype(np.float32)
        assert np.array_equal(out[t], acc)
    # the reference's combine: output[token_ids] += w * expert_out, per expert (model/moe.py:1594)
    ref = torch.zeros(T, D)
    for e in range(E):
        tok = (idx == e).any(-1).nonzero(as_tuple=True)[0]
        pw = (w[tok] * (idx[tok] == e).float()).sum(-1)
        rows = [r["row_of"][t * K + int((idx[t] == e).nonzero()[0])] for t in tok.tolist()]
        ref[tok] += pw[:, None] * torch.from_numpy(y[rows])
    assert np.allclose(out, ref.numpy(), rtol=1e-6, atol=1e-6)


def test_router_logits_matches_reference_linear():
    """oracle.router_logits against the reference's gate: nn.Linear(D, E,
    bias=True) applied to x.float() (model/moe.py:107, :151), plus score_bias
    (:153-154), evaluated in float64 by torch."""
    g = torch.Generator().manual_seed(3)
    T, D, E = 64, 96, 12
    x = torch.randn(T, D, generator=g).bfloat16()
    gate = torch.nn.Linear(D, E, bias=True).double()
    with torch.no_grad():
        gate.weight.copy_(torch.randn(E, D, generator=g) * 0.02)
        gate.bias.fill_(-1.0)
    sb = torch.randn(E, generator=g) * 0.1
    ref = (gate(x.double()) + sb.double()).detach().numpy()
    got = orouting.router_logits(x.float().numpy(), gate.weight.detach().float().numpy(),
                                 gate.bias.detach().float().numpy(), sb.numpy())
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-7)
    # a transposed operand or a dropped bias is caught
    bad = orouting.router_logits(x.float().numpy(), gate.weight.detach().float().numpy())
    assert not np.allclose(bad, ref, atol=1e-3)


def _replay_reference(logits, mask_idx, K):
    """MoERouter._routing_replay_gating (model/moe.py:187-247) as torch ops, float64."""
    train_probs = F.softmax(logits, dim=-1)
    N, E = logits.shape
    full_mask = torch.zeros(N, E, dtype=logits.dtype)
    for k in range(K):
        full_mask.scatter_(1, mask_idx[:, k : k + 1], 1.0)
    masked = train_probs * full_mask
    s = masked.sum(dim=-1, keepdim=True).clamp(min=1e-8)
    return (masked / s).topk(K, dim=-1)


@pytest.mark.parametrize("E,K", [(8, 2), (64, 6), (256, 8)])
def test_replay_gating_matches_reference_ops(E, K):
    g = torch.Generator().manual_seed(E + K)
    logits = torch.randn(300, E, generator=g) * 3
    mask = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(300)])
    rw, ridx = _replay_reference(logits.double(), mask, K)
    w, idx = orouting.replay_gating(logits.numpy(), mask.numpy(), K)
    assert np.array_equal(idx, ridx.numpy())
    assert np.allclose(w, rw.numpy(), rtol=1e-6, atol=1e-9)
    # the replayed experts are exactly the ones selected
    assert all(set(a) == set(b) for a, b in zip(idx.tolist(), mask.tolist()))
    # a permuted mask replays the same routing; a wrong one does not
    w2, idx2 = orouting.replay_gating(logits.numpy(), mask.flip(1).numpy(), K)
    assert np.array_equal(idx2, idx) and np.array_equal(w2, w)


def test_l2_normalize_and_z_loss_match_reference_ops():
    g = torch.Generator().manual_seed(5)
    w = torch.rand(200, 4, generator=g)
    ref = w.double() / (w.double().norm(dim=-1, keepdim=True) + 1e-8)      # model/moe.py:167-170
    assert np.allclose(orouting.l2_normalize(w.numpy()), ref.numpy(), rtol=1e-6)
    logits = torch.randn(2, 128, 16, generator=g) * 4
    zref = torch.logsumexp(logits.double(), dim=-1).square().mean()         # model/moe.py:176-178
    assert abs(orouting.z_loss(logits.reshape(-1, 16).numpy()) - float(zref)) < 1e-9 * float(zref)


def test_score_bias_update_matches_reference_ops():
    """post_batch's fp32 arithmetic (model/moe.py:307-317) as torch ops: bit-exact."""
    g = torch.Generator().manual_seed(6)
    E, K, B, S = 16, 2, 4, 256
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(B * S)]).reshape(B, S, K)
    counts = torch.stack([(idx == e).sum() for e in range(E)])                 # :288-289
    total = torch.tensor(idx.shape[0] * idx.shape[1])                            # :291 (B * S tokens)
    sb = torch.randn(E, generator=g) * 0.1
    gamma = 0.003
    actual = counts.float() / total.float()
    ideal = torch.ones(E) / E
    ref = sb + gamma * (actual - ideal)
    got = orouting.score_bias_update(sb.numpy(), counts.numpy(), int(total), gamma)
    assert np.array_equal(got.view(np.uint32), ref.numpy().view(np.uint32))
    assert np.isclose(actual.sum().item(), K)                                    # fractions sum to K
    assert np.array_equal(orouting.score_bias_update(sb.numpy(), counts.numpy(), 0, gamma), sb.numpy())


def test_topk_nan_first_and_no_duplicates():
    s = np.array([[1, 3, np.nan, 3, -np.inf, -np.inf], [-np.inf] * 6, [np.nan, 0, np.nan, 1, 2, 3]],
                 np.float32)
    idx = orouting.topk_lower_index(s, 6)
    assert idx.tolist() == [[2, 1, 3, 0, 4, 5], [0, 1, 2, 3, 4, 5], [0, 2, 5, 4, 3, 1]]
    t = torch.from_numpy(s).topk(6).indices.numpy()
    assert t[0, 0] == 2 and all(len(set(r)) == 6 for r in t)   # torch: NaN first, no repeats


def _capacity_running_count(idx, E, capacity):
    """Token by token: each slot takes its expert's next rank; a token is kept
    when all its ranks are below the capacity."""
    seen = [0] * E
    keep = []
    for row in np.asarray(idx).tolist():
        ok = True
        for e in set(row):
            if 0 <= e < E:
                ok &= seen[e] < capacity
                seen[e] += 1
        keep.append(ok)
    drops = np.array([max(0, n - capacity) for n in seen], np.int64)
    return np.array(keep, bool), drops


def test_capacity_keep_hand_worked():
    """Expert 0 holds tokens 0, 1, 2, 4; expert 1 tokens 0, 2, 3; expert 2
    tokens 1, 3, 4.  At capacity 2 expert 0 drops 2 and 4, expert 1 drops 3
    (ranked among all its tokens, token 2 included although expert 0 dropped
    it) and expert 2 drops 4."""
    idx = np.array([[0, 1], [0, 2], [1, 0], [2, 1], [0, 2]])
    keep, drops, dropped = orouting.capacity_keep(idx, 3, 2)
    assert keep.tolist() == [True, True, False, False, False]
    assert drops.tolist() == [2, 1, 1] and dropped == 4
    # a capacity of every token keeps all; capacity 0 drops every routed token
    keep, drops, dropped = orouting.capacity_keep(idx, 3, 5)
    assert keep.all() and dropped == 0
    keep, drops, dropped = orouting.capacity_keep(np.array([[0, 1], [-1, 7], [2, 1]]), 3, 0)
    assert keep.tolist() == [False, True, False] and drops.tolist() == [1, 2, 1]


@pytest.mark.parametrize("K,E", [(1, 4), (2, 8), (4, 16)])
def test_capacity_keep_matches_running_counts(K, E):
    T = 3000
    idx = zipf_routing(T, E, K, 1.1, seed=K * 10 + E)[1].numpy().copy()
    idx[::97, 0] = -1                              # out-of-range slots constrain nothing
    counts = np.bincount(idx[idx >= 0], minlength=E)
    for cap in (0, 1, int(T * K / E * 0.8), int(counts.max()) - 1, int(counts.max()), T):
        keep, drops, dropped = orouting.capacity_keep(idx, E, cap)
        rk, rd = _capacity_running_count(idx, E, cap)
        assert np.array_equal(keep, rk) and np.array_equal(drops, rd), cap
        assert dropped == int(rd.sum())
        for e in range(E):                          # no expert keeps more than its capacity
            assert int(((idx == e).any(-1) & keep).sum()) <= cap


def test_adaptive_capacity_hand_worked():
    """T=8 tokens all on expert 0 of 2 (top-1): capacity int(cf * 8 / 2); at cf=1
    the estimated drop rate is 4/8, EMA 0.3 * 0.5 = 0.15 > 1.5 * 0.01, so the
    factor grows 10%; it is clamped at 4 on the way up and at 1 on the way
    down (no drops: the EMA decays below 0.5 * target)."""
    idx = np.zeros((8, 1), np.int64)
    cf, ema, step = orouting.adaptive_capacity_update(1.0, 0.0, 0, idx, 2, 0.01, 0.3)
    assert abs(cf - 1.1) < 1e-12 and abs(ema - 0.15) < 1e-12 and step == 1
    # 8 experts: capacity int(3.9 * 8 / 8) = 3 < 8 tokens, so the factor grows, to the clamp
    cf, ema, step = orouting.adaptive_capacity_update(3.9, 0.0, 0, idx, 8, 0.01, 0.3)
    assert cf == 4.0 and abs(ema - 0.3 * 5 / 8) < 1e-12
    even = np.array([[0], [1]] * 4)
    cf, ema, step = orouting.adaptive_capacity_update(1.02, 0.001, 5, even, 2, 0.01, 0.3)
    assert cf == 1.0 and abs(ema - 0.0007) < 1e-12 and step == 6
    cf, ema, step = orouting.adaptive_capacity_update(2.0, 0.01, 0, even, 2, 0.01, 0.3)
    assert cf == 2.0 and abs(ema - 0.007) < 1e-12               # within [0.5, 1.5] x target: unchanged
