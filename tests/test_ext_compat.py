"""The reference-shaped extension objects (token2tile/operator/deploy_step.py
call sites 343-475) reproduce the operator's own call bit for bit."""
import pytest
import torch

from token2tile_amd import ext_compat


def test_loaders_expose_reference_methods():
    kmm = ext_compat.KmmExt()
    sel = ext_compat.SelectUnionExt()
    att = ext_compat.TileAttnExt()
    for obj, names in ((kmm, ("run", "run_vstats", "run_vstats_gather")),
                       (sel, ("run", "run_split", "run_packed", "run_split_packed")),
                       (att, ("run", "run_planned"))):
        for n in names:
            assert callable(getattr(obj, n))


@pytest.mark.gpu
@pytest.mark.parametrize("split", [False, True])
def test_reference_call_sequence_matches_operator(dev, split):
    from token2tile_amd import deploy_step, ops
    H, N, CQ, C, D = 2, 8192, 64, 2048, 128
    g = torch.Generator(device="cpu").manual_seed(11)
    q, k, v = (torch.randn(H, N, D, generator=g).to(dev, torch.float16) for _ in range(3))
    op = deploy_step.MaskedStepDeploy(H, N, CQ, C=C, D=D, s_frac=0.03, device=dev)
    state = op.init_state(q, k, seed=5)
    st0 = {n: t.clone() for n, t in state.items()}
    ref = op.step(q, k, v, state).clone()

    kmm = ext_compat.load_kmm_ext()
    sel = ext_compat.load_select_union_ext()
    att = ext_compat.load_tile_attn_ext()
    i32, f16 = torch.int32, torch.float16
    QU = ops.project(q, st0["Uq"])
    KU = ops.project(k, st0["Uk"])
    qlab, klab = torch.empty(H, N, dtype=i32, device=dev), torch.empty(H, N, dtype=i32, device=dev)
    cq2 = torch.empty(H, CQ, 32, dtype=f16, device=dev)
    ck2 = torch.empty(H, C, 32, dtype=torch.float32, device=dev)
    qcounts, kcounts = (torch.empty(H, n, dtype=i32, device=dev) for n in (CQ, C))
    qperm, kperm = (torch.empty(H, N, dtype=i32, device=dev) for _ in range(2))
    vp, kp = torch.empty_like(v), torch.empty_like(k)
    sumv = torch.empty(H, C, D, dtype=f16, device=dev)
    lam = torch.empty(H, dtype=torch.float32, device=dev)
    kmm.run(QU, KU, v, st0["cq"], st0["ck"], qlab, cq2, klab, ck2, qcounts, qperm, kcounts,
            kperm, vp, sumv, lam, 0)
    _, cks = ops.centroid_finalize(ck2)
    gl = ops.score(QU, cks)
    unip = torch.empty(H, CQ, C // 32, dtype=i32, device=dev)
    rowcnt = torch.empty(H, N, dtype=i32, device=dev)
    if split:
        sel.run_split_packed(gl, kcounts, qperm, qcounts, (N + CQ - 1) // CQ, op.ns_t, None, unip,
                             rowcnt, None, None, None, None)
    else:
        sel.run_packed(gl, kcounts, qperm, qcounts, op.ns_t, None, unip, rowcnt, None)
    ops.fast_gather(k, kperm, out=kp)
    small_plan = torch.empty(16, dtype=i32, device=dev)  # smaller than the library's plan
    out = torch.empty_like(q)
    att.run_planned(q, kp, vp, qcounts, kcounts, unip.view(torch.uint8).reshape(H, CQ, C // 8),
                    QU, cks, sumv, lam, qlab, qperm, op.tailw_t, out, small_plan, True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # the byte-union entry agrees with the packed bitmap
    bytes_u = torch.empty(H, CQ, C, dtype=torch.uint8, device=dev)
    rowcnt2 = torch.empty_like(rowcnt)
    sel.run(gl, kcounts, qperm, qcounts, op.ns_t, bytes_u, rowcnt2)
    bits = ((unip.view(torch.uint8).unsqueeze(-1) >> torch.arange(8, device=dev, dtype=torch.uint8))
            & 1).reshape(H, CQ, C)
    assert torch.equal(bytes_u, bits) and torch.equal(rowcnt2, rowcnt)
    # a reuse call (rebuild=False) through the same small plan reproduces it
    out2 = torch.empty_like(q)
    att.run_planned(q, kp, vp, qcounts, kcounts, unip.view(torch.uint8).reshape(H, CQ, C // 8),
                    QU, cks, sumv, lam, qlab, qperm, op.tailw_t, out2, small_plan, False)
    vp2, sumv2, lam2 = torch.empty_like(v), torch.empty_like(sumv), torch.empty_like(lam)
    kmm.run_vstats_gather(v, kperm, kcounts, vp2, sumv2, lam2)
    torch.cuda.synchronize()
    assert torch.equal(out2, ref)
    assert torch.equal(vp2, vp) and torch.equal(sumv2, sumv) and torch.equal(lam2, lam)
    sumv3, lam3 = torch.empty_like(sumv), torch.empty_like(lam)
    kmm.run_vstats(vp2, kcounts, sumv3, lam3)
    torch.cuda.synchronize()
    assert torch.equal(sumv3, sumv) and torch.equal(lam3, lam)
