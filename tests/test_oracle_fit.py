"""Pins the oracle's projection fit (S0) by its Eckart-Young invariants:
(Q Uq)(K Uk)^T is the best rank-r approximation of Q K^T in the whitened
metric, and Uq^T Mq Uq = diag(S_r) = Uk^T Mk Uk.  Non-finite input raises."""
import numpy as np
import pytest

from oracle import t2t_oracle as O


def test_online_u_invariants():
    rng = np.random.default_rng(0)
    H, N, D, r = 2, 2000, 128, 32
    A = rng.normal(0, 1, (D, D)) / np.sqrt(D)
    q = (rng.normal(0, 1, (H, N, D)) @ A).astype(np.float32)
    k = (rng.normal(0, 1, (H, N, D)) @ A.T + 0.1 * rng.normal(0, 1, (H, N, D))).astype(np.float32)
    Uq, Uk = O.online_u(q, k, r)
    for h in range(H):
        qd, kd = q[h].astype(np.float64), k[h].astype(np.float64)
        Mq, Mk = qd.T @ qd / N, kd.T @ kd / N
        uq, uk = Uq[h].astype(np.float64), Uk[h].astype(np.float64)
        # whitened singular values of Rq^T Rk, Rq = Mq^(1/2)
        w, V = np.linalg.eigh(Mq)
        Rq = (V * np.sqrt(w)) @ V.T
        w2, V2 = np.linalg.eigh(Mk)
        Rk = (V2 * np.sqrt(w2)) @ V2.T
        S = np.linalg.svd(Rq.T @ Rk, compute_uv=False)[:r]
        assert np.allclose(uq.T @ Mq @ uq, np.diag(S), atol=2e-5 * S[0])
        assert np.allclose(uk.T @ Mk @ uk, np.diag(S), atol=2e-5 * S[0])
        # best rank-r approximation of the bilinear form Mq^(-1/2)... : the
        # product Uq Uk^T equals Rq^-1 (Rq^T Rk)_r Rk^-1
        Rqi, Rki = np.linalg.inv(Rq), np.linalg.inv(Rk)
        U, Sf, Vh = np.linalg.svd(Rq.T @ Rk)
        best = (U[:, :r] * Sf[:r]) @ Vh[:r]
        assert np.allclose(uq @ uk.T, Rqi.T @ best @ Rki.T, atol=1e-4)


def fit_case():
    rng = np.random.default_rng(0)
    H, N, D, r = 2, 2000, 128, 32
    A = rng.normal(0, 1, (D, D)) / np.sqrt(D)
    q = (rng.normal(0, 1, (H, N, D)) @ A).astype(np.float32)
    k = (rng.normal(0, 1, (H, N, D)) @ A.T + 0.1 * rng.normal(0, 1, (H, N, D))).astype(np.float32)
    return q, k, r


@pytest.mark.gpu
def test_operator_online_u_invariants(dev):
    """The operator's fit (Gram + eigh of M^T M on the GPU) satisfies the same
    invariants and gives the oracle's product Uq Uk^T."""
    import torch
    from token2tile_amd.deploy_step import online_u
    q, k, r = fit_case()
    Uq, Uk = (t.cpu().numpy().astype(np.float64) for t in
              online_u(torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev), r))
    Oq, Ok = O.online_u(q, k, r)
    N = q.shape[1]
    for h in range(q.shape[0]):
        qd, kd = q[h].astype(np.float64), k[h].astype(np.float64)
        Mq, Mk = qd.T @ qd / N, kd.T @ kd / N
        S = np.diag(Oq[h].astype(np.float64).T @ Mq @ Oq[h].astype(np.float64))
        assert np.allclose(Uq[h].T @ Mq @ Uq[h], np.diag(S), atol=2e-5 * S[0])
        assert np.allclose(Uk[h].T @ Mk @ Uk[h], np.diag(S), atol=2e-5 * S[0])
        assert np.allclose(Uq[h] @ Uk[h].T, Oq[h].astype(np.float64) @ Ok[h].astype(np.float64).T,
                           atol=1e-4)


def test_online_u_rejects_nonfinite():
    q = np.zeros((1, 10, 128), dtype=np.float32)
    q[0, 3, 4] = np.nan
    with pytest.raises(RuntimeError):
        O.online_u(q, np.zeros_like(q))
