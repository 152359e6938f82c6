"""Prep (RMSNorm + RoPE + f16 KV append) parity on MI355X, and the engine's call sequence:
prep_batch -> prefill for a prompt, then prep -> split -> combine per decoded token, as
src/engine/attention.hip:76-148 orders them, against the oracle run on the same cache.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import report, to_dev, to_host

pytestmark = pytest.mark.gpu

H, KV, D = 16, 2, 256
PROJ = 9216  # [q+gate 8192 | k 512 | v 512]
EPS = 1e-6
ROPE_BASE = 10_000_000.0


def weights(O):
    rng = np.random.default_rng(77)
    q_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    k_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    return q_norm, k_norm, O.inv_freq(ROPE_BASE)


def f16_ulps(a, b):
    """|a - b| in binary16 ulps for same-sign finite values (bit distance)."""
    return np.abs(a.astype(np.int32) - b.astype(np.int32))


@pytest.mark.parametrize("pos", [0, 1, 77, 30000])
def test_prep_matches_oracle(O, attn, torch_mod, ref_kernels, pos):
    torch = torch_mod
    max_ctx = 30001
    proj = O.normal(500 + pos, PROJ)
    qg, k, v = proj[:8192], proj[8192:8704], proj[8704:]
    q_norm, k_norm, inv = weights(O)
    dq = torch.empty(H * D, device="cuda")
    kc = torch.zeros(KV * max_ctx * D, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    dev = [to_dev(torch, a) for a in (qg, k, v, q_norm, k_norm, inv)]
    attn.attn_prep(*dev, kc, vc, dq, pos, max_ctx, EPS)
    torch.cuda.synchronize()
    q_ref, k_ref, v_ref = O.prep_f64(qg, k, v, q_norm, k_norm, inv, pos, EPS)
    st = O.compare(to_host(dq).reshape(H, D), q_ref, atol=1e-5, rtol=1e-5)
    report(f"prep q pos={pos}", st)
    assert st["ok"], st
    kh = to_host(kc).reshape(KV, max_ctx, D)
    vh = to_host(vc).reshape(KV, max_ctx, D)
    assert np.array_equal(vh[:, pos], v_ref)  # V is only rounded
    assert f16_ulps(kh[:, pos], k_ref).max() <= 1
    other = np.ones(max_ctx, bool)
    other[pos] = False
    assert not kh[:, other].any() and not vh[:, other].any()  # nothing else written
    if ref_kernels is not None:  # the reference's own prep kernel, built from its sources
        rq = torch.empty(H * D, device="cuda")
        rk = torch.zeros_like(kc)
        rv = torch.zeros_like(kc)
        torch.cuda.synchronize()
        assert ref_kernels.ref_attn_prep(*[t.data_ptr() for t in dev], rk.data_ptr(),
                                         rv.data_ptr(), rq.data_ptr(), pos, max_ctx, EPS) == 0
        torch.cuda.synchronize()
        st = O.compare(to_host(dq), to_host(rq).astype(np.float64), atol=1e-5, rtol=1e-5)
        assert st["ok"], st
        assert f16_ulps(to_host(rk).reshape(KV, max_ctx, D)[:, pos], kh[:, pos]).max() <= 1


def test_engine_sequence_prefill_then_decode(O, attn, torch_mod):
    """prep_batch + prefill of a 70-token prompt, then 5 decode tokens (prep at pos = len,
    len += 1, split + combine over len) -- every output against the oracle."""
    torch = torch_mod
    P, T, max_ctx = 70, 5, 96
    q_norm, k_norm, inv = weights(O)
    w = [to_dev(torch, a) for a in (q_norm, k_norm, inv)]
    kc = torch.zeros(KV * max_ctx * D, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    kc_h = np.zeros((KV, max_ctx, D), np.uint16)
    vc_h = np.zeros_like(kc_h)
    proj = O.normal(31337, (P + T) * PROJ).reshape(P + T, PROJ)
    # prompt
    dproj = to_dev(torch, proj[:P].ravel())
    dq = torch.empty(P * H * D, device="cuda")
    attn.attn_prep_batch(dproj, dproj[8192:], dproj[8704:], *w, kc, vc, dq, 0, max_ctx, EPS, P,
                         PROJ)
    core = torch.full((P * H * D,), -1.0, device="cuda")
    attn.attn_prefill(dq, dproj, kc, vc, core, 0, P, max_ctx, PROJ)
    torch.cuda.synchronize()
    q_rows = []
    for t in range(P):
        qr, kr, vr = O.prep_f64(proj[t, :8192], proj[t, 8192:8704], proj[t, 8704:], q_norm,
                                k_norm, inv, t, EPS)
        q_rows.append(qr.astype(np.float32))
        kc_h[:, t], vc_h[:, t] = kr, vr
    # the device cache holds the device prep's rounding; check it, then use it for the oracle
    kd = to_host(kc).reshape(KV, max_ctx, D)
    assert f16_ulps(kd[:, :P], kc_h[:, :P]).max() <= 1
    st = O.compare(to_host(dq).reshape(P, H, D), np.stack(q_rows).astype(np.float64), atol=1e-5,
                   rtol=1e-5)
    assert st["ok"], st
    ref = O.prefill_f64(to_host(dq), proj[:P].ravel(), PROJ, kd.ravel(),
                        to_host(vc), 0, max_ctx, np.arange(P))
    st = O.compare(to_host(core).reshape(P, H, D), ref)
    report("engine prefill", st)
    assert st["ok"], st
    # decode tokens
    sc = attn.DecodeScratch(60)
    q1 = torch.empty(H * D, device="cuda")
    out = torch.empty(H * D, device="cuda")
    for i in range(T):
        pos = P + i
        dp = to_dev(torch, proj[pos])
        attn.attn_prep(dp[:8192], dp[8192:8704], dp[8704:], *w, kc, vc, q1, pos, max_ctx, EPS)
        attn.attn_decode(q1, dp[:8192], kc, vc, out, sc, pos + 1, max_ctx)
        torch.cuda.synchronize()
        ref = O.decode_f64(to_host(q1), proj[pos, :8192], to_host(kc), to_host(vc), pos + 1,
                           max_ctx)
        st = O.compare(to_host(out).reshape(H, D), ref)
        report(f"engine decode len={pos + 1}", st)
        assert st["ok"], st
