"""Pins the CPU oracle (oracle/) before anything is compared against it.

Every oracle function is checked by a route that does not retype its formula:
  forward   -- a dense-GEMM formulation through torch.matmul (float64), a hand-computed known
               answer, one-hot inputs (closed form), mean = sum / n_g, masking of padded slots;
  backward  -- torch autograd of the dense formulation, float64 central differences;
  adam      -- torch.optim.AdamW / Adam (library) and the step-1 closed form;
  partition -- the invariants of the reference's test_partition_enumerates_exactly_H;
  xedges    -- a brute-force per-feature enumeration written with plain Python loops.
Each check is chosen so that a dropped term, wrong sign, wrong index or transposed operand fails.
"""
import numpy as np
import pytest
import torch

from conftest import assert_close, rel_err


def random_problem(rng, B, D, G, S, K, ragged=True, bias_std=0.3):
    counts = rng.integers(max(1, S // 2), S + 1, size=G).astype(np.int32) if ragged else np.full(G, S, np.int32)
    idx = np.zeros((G * S, K), np.int32)
    w = np.zeros((G * S, K), np.float32)
    b = np.zeros(G * S, np.float32)
    for g in range(G):
        for s in range(counts[g]):
            n = g * S + s
            idx[n] = np.sort(rng.choice(D, K, replace=False))
            w[n] = rng.standard_normal(K).astype(np.float32) / np.sqrt(K)
            b[n] = rng.standard_normal() * bias_std
    x = rng.standard_normal((B, D)).astype(np.float32)
    return x, idx, w, b, counts


def _act(z, act):
    """The neuron activation through torch's own ops: relu, exact (erf) GELU, identity."""
    if act == "relu":
        return torch.relu(z)
    if act == "gelu":
        return torch.nn.functional.gelu(z, approximate="none")
    return z


def dense_forward(x, idx, w, b, counts, S, act, pool):
    """float64 torch formulation through a dense [N, D] weight matrix and torch.matmul."""
    x = torch.as_tensor(x, dtype=torch.float64)
    G = len(counts)
    N, K = idx.shape
    D = x.shape[1]
    valid = (torch.arange(S)[None, :] < torch.as_tensor(counts)[:, None]).reshape(-1)
    Wd = torch.zeros(N, D, dtype=torch.float64)
    Wd.scatter_(1, torch.as_tensor(idx, dtype=torch.int64), torch.as_tensor(w, dtype=torch.float64))
    Wd = Wd * valid[:, None]
    z = torch.matmul(x, Wd.T) + torch.as_tensor(b, dtype=torch.float64) * valid
    a = _act(z, act)
    a = a * valid
    s = a.reshape(x.shape[0], G, S).sum(-1)
    return s / torch.as_tensor(counts, dtype=torch.float64) if pool == "mean" else s


@pytest.mark.parametrize("act", ["relu", "identity", "gelu"])
@pytest.mark.parametrize("pool", ["mean", "sum"])
@pytest.mark.parametrize("B,D,G,S,K", [(3, 16, 2, 32, 8), (5, 40, 3, 64, 8), (2, 64, 2, 32, 16)])
def test_forward_matches_dense_gemm(oracle, act, pool, B, D, G, S, K):
    rng = np.random.default_rng(1)
    x, idx, w, b, counts = random_problem(rng, B, D, G, S, K)
    got = oracle.forward(x, idx, w, b, counts, S, act, pool)
    want = dense_forward(x, idx, w, b, counts, S, act, pool).numpy()
    assert_close(got, want, rtol=1e-12, atol=1e-12, what="forward")


def test_forward_known_answer(oracle):
    # neuron 0: x0*1 + x2*2 + 0.5 = 7.5 ; neuron 1: -x1 + 0.25*x3 - 0.25 = -1.25
    x = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    idx = np.array([[0, 2], [1, 3]], np.int32)
    w = np.array([[1.0, 2.0], [-1.0, 0.25]], np.float32)
    b = np.array([0.5, -0.25], np.float32)
    c2 = np.array([2], np.int32)
    assert oracle.forward(x, idx, w, b, c2, 2, "relu", "sum")[0, 0] == 7.5
    assert oracle.forward(x, idx, w, b, c2, 2, "relu", "mean")[0, 0] == 3.75
    assert oracle.forward(x, idx, w, b, c2, 2, "identity", "sum")[0, 0] == 6.25
    assert oracle.forward(x, idx, w, b, c2, 2, "identity", "mean")[0, 0] == 3.125
    # neuron 1 padded away: only neuron 0 counts
    assert oracle.forward(x, idx, w, b, np.array([1], np.int32), 2, "identity", "mean")[0, 0] == 7.5


def test_forward_one_hot_inputs(oracle):
    rng = np.random.default_rng(2)
    B, D, G, S, K = 24, 24, 3, 32, 8
    _, idx, w, b, counts = random_problem(rng, B, D, G, S, K, bias_std=0.0)
    x = np.eye(D, dtype=np.float32)  # token d is the one-hot vector e_d
    got = oracle.forward(x, idx, w, b, counts, S, "identity", "sum")
    want = np.zeros((D, G))
    for g in range(G):
        for s in range(counts[g]):
            n = g * S + s
            for k in range(K):
                want[idx[n, k], g] += w[n, k]
    assert_close(got, want, rtol=1e-12, atol=1e-12, what="one-hot")


def test_mean_is_sum_over_count_and_padding_is_masked(oracle):
    rng = np.random.default_rng(3)
    B, D, G, S, K = 4, 32, 3, 64, 8
    x, idx, w, b, counts = random_problem(rng, B, D, G, S, K)
    s = oracle.forward(x, idx, w, b, counts, S, "relu", "sum")
    m = oracle.forward(x, idx, w, b, counts, S, "relu", "mean")
    assert_close(m * counts[None, :], s, rtol=1e-14, atol=0, what="mean*n")
    # garbage in padded slots must not change anything
    w2, b2, idx2 = w.copy(), b.copy(), idx.copy()
    for g in range(G):
        for sl in range(counts[g], S):
            n = g * S + sl
            w2[n] = 100.0
            b2[n] = 50.0
            idx2[n] = np.arange(K)
    assert np.array_equal(oracle.forward(x, idx2, w2, b2, counts, S, "relu", "sum"), s)


@pytest.mark.parametrize("act", ["relu", "identity", "gelu"])
@pytest.mark.parametrize("pool", ["mean", "sum"])
def test_backward_matches_autograd(oracle, act, pool):
    rng = np.random.default_rng(4)
    B, D, G, S, K = 6, 48, 3, 32, 8
    x, idx, w, b, counts = random_problem(rng, B, D, G, S, K)
    dy = rng.standard_normal((B, G)).astype(np.float32)
    dW, db, dX = oracle.backward(x, idx, w, b, counts, S, dy, act, pool)
    # autograd through the dense formulation
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    N = G * S
    valid = (torch.arange(S)[None, :] < torch.as_tensor(counts)[:, None]).reshape(-1)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    Wd = torch.zeros(N, D, dtype=torch.float64).scatter(1, torch.as_tensor(idx, dtype=torch.int64), wt)
    z = torch.matmul(xt, (Wd * valid[:, None]).T) + bt * valid
    a = (_act(z, act)) * valid
    s = a.reshape(B, G, S).sum(-1)
    y = s / torch.as_tensor(counts, dtype=torch.float64) if pool == "mean" else s
    (y * torch.as_tensor(dy, dtype=torch.float64)).sum().backward()
    assert_close(dX, xt.grad.numpy(), rtol=1e-12, atol=1e-12, what="dX")
    assert_close(dW, (wt.grad * valid[:, None]).numpy(), rtol=1e-12, atol=1e-12, what="dW")
    assert_close(db, (bt.grad * valid).numpy(), rtol=1e-12, atol=1e-12, what="db")


def dense_z(x, idx, w, b, counts, S):
    """float64 z [B, G, S] and slot validity [G, S] through a dense weight matrix (torch.matmul)."""
    x = torch.as_tensor(x, dtype=torch.float64)
    G = len(counts)
    N, K = idx.shape
    valid = torch.arange(S)[None, :] < torch.as_tensor(counts)[:, None]
    Wd = torch.zeros(N, x.shape[1], dtype=torch.float64)
    Wd.scatter_(1, torch.as_tensor(idx, dtype=torch.int64), torch.as_tensor(w, dtype=torch.float64))
    z = torch.matmul(x, Wd.T) + torch.as_tensor(b, dtype=torch.float64)
    return z.reshape(x.shape[0], G, S), valid


@pytest.mark.parametrize("act", ["identity", "relu", "gelu"])
@pytest.mark.parametrize("B,D,G,S,K", [(4, 16, 3, 32, 8), (3, 40, 2, 64, 16)])
def test_forward_max_matches_torch_argmax(oracle, act, B, D, G, S, K):
    # pytorch_reference.py:61-67: am = where(mask, act(z), -inf); winner = argmax (first maximum)
    rng = np.random.default_rng(11)
    x, idx, w, b, counts = random_problem(rng, B, D, G, S, K)
    z, valid = dense_z(x, idx, w, b, counts, S)
    a = _act(z, act)
    am = torch.where(valid[None], a, torch.tensor(float("-inf"), dtype=torch.float64))
    want_pre, want_win = am.max(-1).values.numpy(), am.argmax(-1).numpy()
    pre, win, gap = oracle.forward_max(x, idx, w, b, counts, S, act)
    assert_close(pre, want_pre, rtol=1e-12, atol=1e-12, what="max pre")
    assert (win == want_win).all()
    assert (gap > 0).all() or act == "relu"  # relu: several zeros tie at the maximum 0


def test_forward_max_ties_go_to_the_smaller_slot(oracle):
    # slots 1 and 3 both reach z = 2 (x = [1, 1]); slot 0 reaches 1; slot 2 is padded away (n_g = 4
    # but its z = 5 would win if it counted) -- winner 1, the first maximum
    x = np.array([[1.0, 1.0]], np.float32)
    idx = np.array([[0, 1], [0, 1], [0, 1], [0, 1], [0, 1]], np.int32)
    w = np.array([[0.5, 0.5], [1.0, 1.0], [2.5, 2.5], [1.0, 1.0], [9.0, 9.0]], np.float32)
    b = np.zeros(5, np.float32)
    pre, win, gap = oracle.forward_max(x, idx, w, b, np.array([4], np.int32), 5, "identity")
    assert pre[0, 0] == 5.0 and win[0, 0] == 2  # slot 2 counts (n_g = 4): z = 5
    pre, win, gap = oracle.forward_max(x, idx, w[[0, 1, 3, 2, 4]], b, np.array([3], np.int32), 5, "identity")
    assert pre[0, 0] == 2.0 and win[0, 0] == 1 and gap[0, 0] == 0.0  # slots 1, 2 tie at 2; slot 3 (z 5) padded
    # relu with every z <= 0: all activations are 0, the first slot wins
    pre, win, _ = oracle.forward_max(-x, idx, w, b, np.array([4], np.int32), 5, "relu")
    assert pre[0, 0] == 0.0 and win[0, 0] == 0


@pytest.mark.parametrize("act", ["identity", "relu", "gelu"])
def test_backward_max_matches_autograd(oracle, act):
    # the gradient reaches only the winner (autograd of am.gather(winner), pytorch_reference.py:61-67)
    rng = np.random.default_rng(12)
    B, D, G, S, K = 5, 24, 3, 32, 8
    x, idx, w, b, counts = random_problem(rng, B, D, G, S, K)
    dy = rng.standard_normal((B, G)).astype(np.float32)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    z = (xt[:, torch.as_tensor(idx, dtype=torch.int64)] * wt).sum(-1) + bt  # [B, N]
    a = _act(z, act)
    valid = (torch.arange(S)[None, :] < torch.as_tensor(counts)[:, None]).reshape(-1)
    am = torch.where(valid[None], a, torch.tensor(float("-inf"), dtype=torch.float64)).reshape(B, G, S)
    win = am.detach().argmax(-1, keepdim=True)
    pooled = am.gather(-1, win).squeeze(-1)
    (pooled * torch.as_tensor(dy, dtype=torch.float64)).sum().backward()
    dW, db, dX = oracle.backward(x, idx, w, b, counts, S, dy, act, "max")
    assert_close(dW, wt.grad.numpy(), rtol=1e-12, atol=1e-12, what="dW")
    assert_close(db, bt.grad.numpy(), rtol=1e-12, atol=1e-12, what="db")
    assert_close(dX, xt.grad.numpy(), rtol=1e-12, atol=1e-12, what="dX")
    assert (np.count_nonzero(db.reshape(G, S), axis=1) <= B).all()  # at most one winner per token


def _topk_reference(x, idx, w, b, counts, S, k, act):
    """The reference's formula (pytorch_reference.py:68-77) on float64 tensors with autograd."""
    B, G = x.shape[0], len(counts)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    z = ((xt[:, torch.as_tensor(idx, dtype=torch.int64)] * wt).sum(-1) + bt).reshape(B, G, S)
    a = _act(z, act)
    mask = (torch.arange(S)[None, :] < torch.as_tensor(counts)[:, None])[None].expand_as(z)
    count = mask.sum(-1).to(z.dtype)
    zm = torch.where(mask, z, torch.tensor(float("-inf"), dtype=torch.float64))
    order = torch.sort(zm.detach(), dim=-1, descending=True, stable=True).indices[..., :k]
    sel_valid = torch.arange(k)[None, None, :] < count[..., None]
    vals = a.gather(-1, order)
    kk = torch.clamp(count, max=k)
    pooled = torch.where(sel_valid, vals, torch.zeros_like(vals)).sum(-1) / kk
    return pooled, torch.where(sel_valid, order, torch.full_like(order, -1)), (xt, wt, bt)


@pytest.mark.parametrize("act", ["identity", "relu", "gelu"])
@pytest.mark.parametrize("k", [1, 4, 16, 64])
def test_forward_topk_matches_reference_formula(oracle, act, k):
    rng = np.random.default_rng(13)
    B, D, G, S, K = 4, 40, 3, 64, 8  # ragged pools of 32-64 slots (k <= S, as the reference assumes)
    x, idx, w, b, counts = random_problem(rng, B, D, G, S, K)
    want_pre, want_slots, _ = _topk_reference(x, idx, w, b, counts, S, k, act)
    pre, slots, gap = oracle.forward_topk(x, idx, w, b, counts, S, k, act)
    assert_close(pre, want_pre.detach().numpy(), rtol=1e-12, atol=1e-12, what="topk pre")
    assert (slots == want_slots.numpy()).all()
    assert (gap > 0).all()


def test_forward_topk_ties_go_to_the_smaller_slot(oracle):
    # z = 3, 5, 5, 3, 9 (slot 4 padded away): k = 2 takes slots 1, 2; k = 3 takes 1, 2, 0 (0 before 3)
    x = np.array([[1.0, 1.0]], np.float32)
    idx = np.array([[0, 1]] * 5, np.int32)
    w = np.array([[1.5, 1.5], [2.5, 2.5], [2.5, 2.5], [1.5, 1.5], [4.5, 4.5]], np.float32)
    b = np.zeros(5, np.float32)
    c4 = np.array([4], np.int32)
    pre, slots, gap = oracle.forward_topk(x, idx, w, b, c4, 5, 2)
    assert pre[0, 0] == 5.0 and slots[0, 0].tolist() == [1, 2]
    pre, slots, gap = oracle.forward_topk(x, idx, w, b, c4, 5, 4)
    assert pre[0, 0] == 4.0 and slots[0, 0].tolist() == [1, 2, 0, 3] and gap[0, 0] == np.inf
    pre, slots, _ = oracle.forward_topk(x, idx, w, b, c4, 5, 8)  # short pool: kk = 4, the rest -1
    assert pre[0, 0] == 4.0 and slots[0, 0].tolist() == [1, 2, 0, 3, -1, -1, -1, -1]
    _, _, gap = oracle.forward_topk(x, idx, w, b, c4, 5, 3)
    assert gap[0, 0] == 0.0  # slot 0 and slot 3 tie at the boundary


@pytest.mark.parametrize("act", ["identity", "relu", "gelu"])
@pytest.mark.parametrize("k", [2, 8])
def test_backward_topk_matches_autograd(oracle, act, k):
    rng = np.random.default_rng(14)
    B, D, G, S, K = 5, 24, 3, 32, 8
    x, idx, w, b, counts = random_problem(rng, B, D, G, S, K)
    dy = rng.standard_normal((B, G)).astype(np.float32)
    pooled, _, (xt, wt, bt) = _topk_reference(x, idx, w, b, counts, S, k, act)
    (pooled * torch.as_tensor(dy, dtype=torch.float64)).sum().backward()
    dW, db, dX = oracle.backward_topk(x, idx, w, b, counts, S, dy, k, act)
    assert_close(dW, wt.grad.numpy(), rtol=1e-12, atol=1e-12, what="dW")
    assert_close(db, bt.grad.numpy(), rtol=1e-12, atol=1e-12, what="db")
    assert_close(dX, xt.grad.numpy(), rtol=1e-12, atol=1e-12, what="dX")


@pytest.mark.parametrize("act", ["identity", "relu", "gelu"])
def test_backward_events_of_the_own_selection_is_the_pooling_backward(oracle, act):
    rng = np.random.default_rng(15)
    B, D, G, S, K = 4, 32, 3, 40, 8
    x, idx, w, b, counts = random_problem(rng, B, D, G, S, K)
    dy = rng.standard_normal((B, G)).astype(np.float32)
    _, win, _ = oracle.forward_max(x, idx, w, b, counts, S, act)
    got = oracle.backward_events(x, idx, w, b, counts, S, dy, win, act)[:3]
    for g_, w_ in zip(got, oracle.backward(x, idx, w, b, counts, S, dy, act, "max")):
        assert_close(g_, w_, rtol=1e-14, atol=1e-14, what="events == max backward")
    for k in (2, 8, 64):
        _, sl, _ = oracle.forward_topk(x, idx, w, b, counts, S, k, act)
        got = oracle.backward_events(x, idx, w, b, counts, S, dy, sl, act, topk=True)[:3]
        for g_, w_ in zip(got, oracle.backward_topk(x, idx, w, b, counts, S, dy, k, act)):
            assert_close(g_, w_, rtol=1e-14, atol=1e-14, what=f"events == top-{k} backward")


def test_backward_accumulates_and_finite_differences(oracle):
    rng = np.random.default_rng(5)
    B, D, G, S, K = 3, 20, 2, 32, 8
    x, idx, w, b, counts = random_problem(rng, B, D, G, S, K)
    dy = rng.standard_normal((B, G)).astype(np.float32)
    dW, db, dX = oracle.backward(x, idx, w, b, counts, S, dy, "identity", "mean")
    # directional derivative along a random input direction v (identity activation: exact)
    v = rng.standard_normal((B, D))
    h = 1e-3

    def f(xx):
        return float((oracle.forward(xx.astype(np.float32), idx, w, b, counts, S, "identity", "mean") * dy).sum())

    fd = (f(x + h * v) - f(x - h * v)) / (2 * h)
    assert abs(fd - float((dX * v).sum())) < 1e-3 * max(1.0, abs(fd))
    # the bias gradient of a valid neuron is sum_b dy[b, g] / n_g
    g0 = 1
    assert abs(db[g0 * S] - dy[:, g0].astype(np.float64).sum() / counts[g0]) < 1e-12


def _torch_adamw(p0, grads, lr, b1, b2, eps, wd):
    q = torch.nn.Parameter(torch.tensor(p0))
    opt = torch.optim.AdamW([q], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    for g in grads:
        q.grad = torch.tensor(g)
        opt.step()
    return q.detach().numpy()


@pytest.mark.parametrize("wd", [0.0, 0.1])
def test_adam_matches_torch_adamw(oracle, wd):
    rng = np.random.default_rng(6)
    n = 4099
    p0 = rng.standard_normal(n).astype(np.float32)
    grads = [rng.standard_normal(n).astype(np.float32) for _ in range(5)]
    p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for t, g in enumerate(grads, 1):
        gg = g.copy()
        oracle.adam(p, gg, m, v, 1e-2, 0.9, 0.999, 1e-8, wd, t)
        assert not gg.any(), "fused zero_grad"
    want = _torch_adamw(p0, grads, 1e-2, 0.9, 0.999, 1e-8, wd)
    # The reference evaluates (1 - beta) in fp32 (optim.py:44-45: fl(1 - fl(0.999)) is 1.3e-5
    # off 0.001) while torch uses the double constant, so the two fp32 recurrences drift apart by
    # ~1e-5 of each update; a dropped term or a wrong bias correction moves p by ~lr per step.
    assert np.abs(p - want).max() < 1e-4 * 1e-2 * len(grads)
    assert rel_err(p, want) < 1e-6


def test_adam_step1_closed_form(oracle):
    rng = np.random.default_rng(7)
    n = 1000
    p0 = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    oracle.adam(p, g.copy(), m, v, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1)
    want = p0.astype(np.float64) - 1e-3 * g / (np.abs(g) + 1e-8)
    assert_close(p, want, rtol=1e-6, atol=1e-7, what="step 1")
    assert_close(m, 0.1 * g.astype(np.float64), rtol=1e-6, atol=0, what="m")
    # (1 - beta2) is formed in fp32 from fl(0.999): 1.3e-5 below 0.001 (see the AdamW test)
    assert_close(v, 0.001 * g.astype(np.float64) ** 2, rtol=2e-5, atol=0, what="v")


def test_adam_bf16_moments_are_rounded_like_torch(oracle):
    rng = np.random.default_rng(8)
    n = 2048
    p = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    oracle.adam(p, g.copy(), m, v, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, moments_bf16=True)
    m_fp32 = (np.float32(0.9) * np.float32(0) + np.float32(0.1) * g).astype(np.float32)
    want = torch.tensor(m_fp32).to(torch.bfloat16).float().numpy()
    assert np.array_equal(m, want)


@pytest.mark.parametrize("H,G", [(100_000_000, 1024), (5000, 16), (1000, 7), (4_194_304, 4096)])
def test_partition_enumerates_exactly_H(oracle, H, G):
    counts, offsets, S = oracle.partition(H, G)
    assert int(counts.sum()) == H
    assert offsets[0] == 0
    assert np.array_equal(offsets[1:], offsets[:-1] + counts[:-1])
    assert int(counts.max() - counts.min()) <= 1
    assert S >= counts.max() and S % 32 == 0


def _xedges_bruteforce(idx, counts, S, D, Fw, US):
    G = len(counts)
    P = -(-S // US)
    K = idx.shape[1]
    out = []  # (F, u, f_local, eid, n, k)
    for F in range(-(-D // Fw)):
        for u in range(G * P):
            g, piece = divmod(u, P)
            for f in range(Fw):
                d = F * Fw + f
                for s in range(piece * US, min((piece + 1) * US, counts[g])):
                    n = g * S + s
                    for k in range(K):
                        if idx[n, k] == d:
                            out.append((F, u, f, n * K + k, n, k))
    return out


@pytest.mark.parametrize("D,G,S,K,Fw,US", [(40, 3, 32, 8, 16, 1024), (64, 2, 96, 8, 16, 32), (48, 2, 64, 16, 16, 64)])
def test_xedges_matches_bruteforce(oracle, D, G, S, K, Fw, US):
    rng = np.random.default_rng(9)
    _, idx, _, _, counts = random_problem(rng, 1, D, G, S, K)
    e = oracle.xedges(idx, counts, S, D, Fw, US)
    want = _xedges_bruteforce(idx, counts, S, D, Fw, US)
    assert len(e["rec"]) == len(want) == int(counts.sum()) * K
    P = -(-S // US)
    got = []
    for F in range(e["FR"]):
        for si in range(e["seg_ptr"][F], e["seg_ptr"][F + 1]):
            u = int(e["seg_unit"][si])
            g, piece = divmod(u, P)
            prev_f = None
            for j in range(e["seg_begin"][si], e["seg_begin"][si + 1]):
                r = int(e["rec"][j])
                el, f, newf = (r & 0xFFFF) >> 2, (r >> 16) & 0xFF, r >> 31
                assert r & 3 == 0 and (r >> 24) & 0x7F == 0
                assert newf == (prev_f is not None and f != prev_f)
                prev_f = f
                nl, k = divmod(el, K)
                n = g * S + piece * US + nl
                got.append((F, u, f, n * K + k, n, k))
    assert got == want


def _dense_pool_torch(x, idx, w, b, counts, S, pool, param, act):
    """The reference's pooling formulas (pytorch_reference.py:80-100) on the dense z of a small
    layer, float64 torch, differentiable in x, w, b."""
    import torch

    G = len(counts)
    xg = x[:, torch.as_tensor(idx, dtype=torch.long)]
    z = (xg * w).sum(-1) + b  # [B, G*S]
    z = z.view(x.shape[0], G, S)
    a = _act(z, "relu" if pool == "power_mean" else act)
    mask = torch.arange(S)[None, :] < torch.as_tensor(counts)[:, None]
    n = torch.as_tensor(counts, dtype=torch.float64)
    if pool == "logmeanexp":
        u = torch.where(mask, a / param, torch.tensor(float("-inf"), dtype=torch.float64))
        return param * (torch.logsumexp(u, -1) - torch.log(n))
    if pool == "power_mean":
        am = torch.where(mask, a, torch.zeros_like(a))
        m = am.amax(-1, keepdim=True)
        safe = torch.where(m > 0, m, torch.ones_like(m))
        s = ((am / safe) ** param).sum(-1) / n
        return torch.where(m.squeeze(-1) > 0, safe.squeeze(-1) * s ** (1.0 / param), torch.zeros_like(s))
    u = torch.where(mask, param * a, torch.tensor(float("-inf"), dtype=torch.float64))
    return (torch.softmax(u, -1) * torch.where(mask, a, torch.zeros_like(a))).sum(-1)


@pytest.mark.parametrize("pool,param,act", [("logmeanexp", 1.0, "identity"), ("logmeanexp", 0.3, "relu"),
                                            ("logmeanexp", 0.7, "gelu"),
                                            ("power_mean", 2.0, "relu"), ("power_mean", 3.5, "relu"),
                                            ("softmax_weighted", 1.0, "identity"), ("softmax_weighted", 2.5, "relu"),
                                            ("softmax_weighted", 1.5, "gelu")])
def test_smooth_pools_match_torch_formulas_and_autograd(oracle, pool, param, act):
    """Forward against the reference's pooling formulas in float64 torch, backward against torch
    autograd of them (dW, db, dX), on ragged pools (padded slots)."""
    import torch

    B, D, G, S, K = 5, 40, 4, 16, 8
    rng = np.random.default_rng(7)
    x = rng.standard_normal((B, D)).astype(np.float32)
    idx = np.stack([np.sort(rng.choice(D, K, replace=False)) for _ in range(G * S)]).astype(np.int32)
    w = (rng.standard_normal((G * S, K)) / 3).astype(np.float32)
    b = (rng.standard_normal(G * S) * 0.3).astype(np.float32)
    counts = np.array([16, 11, 5, 16], np.int32)
    dy = rng.standard_normal((B, G)).astype(np.float32)
    pre, lse, mag = oracle.forward_smooth(x, idx, w, b, counts, S, pool, param, act)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    want = _dense_pool_torch(xt, idx, wt, bt, counts, S, pool, param, act)
    np.testing.assert_allclose(pre, want.detach().numpy(), rtol=1e-12, atol=1e-12)
    (want * torch.tensor(dy, dtype=torch.float64)).sum().backward()
    dW, db, dX, _ = oracle.backward_smooth(x, idx, w, b, counts, S, dy, pool, param, act)
    valid = (np.arange(S)[None, :] < counts[:, None]).reshape(-1)
    np.testing.assert_allclose(dX, xt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dW[valid], wt.grad.numpy()[valid], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db[valid], bt.grad.numpy()[valid], rtol=1e-10, atol=1e-12)
    assert not dW[~valid].any() and not db[~valid].any()
    if pool != "power_mean":  # L2 = log2 sum 2^(u), u = a * scale
        sc = np.log2(np.e) / param if pool == "logmeanexp" else np.log2(np.e) * param
        np.testing.assert_allclose(lse, (pre * sc + np.log2(counts)) if pool == "logmeanexp" else lse, rtol=1e-12)


def test_smooth_backward_finite_differences(oracle):
    """Central differences of the float64 oracle forward give its backward (softmax-weighted)."""
    B, D, G, S, K = 2, 12, 2, 8, 8
    rng = np.random.default_rng(3)
    x = rng.standard_normal((B, D)).astype(np.float32)
    idx = np.stack([np.sort(rng.choice(D, K, replace=False)) for _ in range(G * S)]).astype(np.int32)
    w = (rng.standard_normal((G * S, K)) / 3).astype(np.float32)
    b = (rng.standard_normal(G * S) * 0.3).astype(np.float32)
    counts = np.array([8, 6], np.int32)
    dy = np.ones((B, G), np.float32)
    _, db, _, _ = oracle.backward_smooth(x, idx, w, b, counts, S, dy, "softmax_weighted", 1.7, "identity")
    h = 1e-3
    for n in (0, 3, 9, 13):
        bp, bm = b.copy(), b.copy()
        bp[n] += h
        bm[n] -= h
        fp = oracle.forward_smooth(x, idx, w, bp, counts, S, "softmax_weighted", 1.7)[0].sum()
        fm = oracle.forward_smooth(x, idx, w, bm, counts, S, "softmax_weighted", 1.7)[0].sum()
        # bias steps of 1e-3 are exact in fp32 only approximately: compare at the 1e-5 level
        assert abs((fp - fm) / (2 * h) - db[n]) < 1e-4 * max(1.0, abs(db[n]))
