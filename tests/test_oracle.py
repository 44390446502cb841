"""Pin the CPU oracle (runs without a GPU).

The reference holds no golden vectors for this path, so each oracle function is
pinned by an independent route: an installed library implementation, an fp64
per-element loop, a closed form, or an invariant of the mathematics.
"""
import math

import pytest
import torch

import oracle
from oracle.v4_ref import _heads

N = 128


def _small(seed=0, b=3, H=8, P=16, G=2, rotation=True, dt_min=0.0):
    gen = torch.Generator().manual_seed(seed)
    prm = oracle.make_layer_params(H, P, N, G, gen, rotation=rotation, dt_min=dt_min)
    S0 = oracle.make_state(b, H, P, N, gen)
    return gen, prm, S0


# --------------------------------------------------------------------------- rotation
def test_make_rotation_is_orthogonal_with_positive_qr_diagonal():
    gen = torch.Generator().manual_seed(3)
    R = oracle.make_rotation(4, N, gen).double()
    eye = torch.eye(N, dtype=torch.float64)
    assert torch.allclose(R @ R.transpose(-1, -2), eye.expand(4, N, N), atol=1e-6)
    # the sign fix (Q * sign(diag(R_qr))) makes R the Q of the unique QR of the
    # Gaussian W with a positive triangular diagonal: R^T W is upper triangular, diag > 0
    W = torch.randn(4, N, N, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    T = R.transpose(-1, -2) @ W
    assert torch.allclose(torch.tril(T, -1), torch.zeros_like(T), atol=1e-5)
    assert bool((torch.diagonal(T, dim1=-2, dim2=-1) > 0).all())


def test_rotate_is_R_times_vector_per_group():
    gen = torch.Generator().manual_seed(4)
    R = oracle.make_rotation(3, N, gen)
    X = torch.randn(5, 3, N, generator=gen)
    got = oracle.rotate(X, R)
    for g in range(3):  # B'[m] = sum_n R[g][m][n] B[n]  (a transposed R fails here)
        want = X[:, g, :].double() @ R[g].double().T
        assert torch.allclose(got[:, g].double(), want, atol=1e-5)
    assert oracle.rotate(X, None) is X


def test_softplus_dt_closed_form_and_clamp():
    x = torch.tensor([[-30.0, -2.0, 0.0, 1.5, 19.0, 25.0]])
    bias = torch.tensor([0.1, -0.2, 0.3, 0.0, 0.5, 1.0])
    got = oracle.softplus_dt(x, bias)
    v = (x + bias).double()
    want = torch.where(v > 20, v, torch.log1p(torch.exp(v)))
    assert torch.allclose(got.double(), want, rtol=1e-6, atol=1e-12)
    got2 = oracle.softplus_dt(x, bias, dt_min=0.05)
    assert float(got2.min()) >= 0.05 and torch.equal(got2[got2 > 0.05], got[got > 0.05])


# --------------------------------------------------------------------------- fresh step
def test_fresh_step_matches_transformers_selective_state_update():
    """Installed transformers' mamba2_selective_state_update (an independent
    implementation of the same recurrence), fed fp32-upcast inputs."""
    M = pytest.importorskip("transformers.models.nemotron_h.modeling_nemotron_h")
    gen, prm, S0 = _small(seed=5, b=2, H=8, P=16, G=2)
    b, H, P, G = 2, 8, 16, 2
    S1, S2 = S0.clone(), S0.clone()
    for _ in range(6):
        x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
        y1 = oracle.fresh_step(S1, x, B, C, dt, prm)
        Bp, Cp = oracle.rotate(B.float(), prm.R), oracle.rotate(C.float(), prm.R)
        y2 = M.mamba2_selective_state_update(
            S2, x.float(), dt.float()[..., None].expand(-1, -1, P), prm.A[:, None, None].expand(H, P, N), Bp, Cp,
            prm.D[:, None].expand(H, P), dt_bias=prm.dt_bias[:, None].expand(H, P), dt_softplus=True)
        assert torch.allclose(y1, y2, rtol=1e-5, atol=1e-6)
    assert torch.allclose(S1, S2, rtol=1e-5, atol=1e-7)


def test_fresh_step_matches_fp64_elementwise_loop():
    gen, prm, S0 = _small(seed=6, b=2, H=4, P=8, G=2)
    b, H, P, G = 2, 4, 8, 2
    HG = H // G
    x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
    S = S0.clone().double()
    y = oracle.fresh_step(S, x, B, C, dt, prm.to(torch.float64), dtype=torch.float64)
    Sw = S0.double()
    R = prm.R.double()
    for i in range(b):
        for h in range(H):
            g = h // HG
            Bp = [sum(float(R[g, m, n]) * float(B[i, g, n]) for n in range(N)) for m in range(N)]
            Cp = [sum(float(R[g, m, n]) * float(C[i, g, n]) for n in range(N)) for m in range(N)]
            v = float(dt[i, h]) + float(prm.dt_bias[h])
            d = math.log1p(math.exp(v))
            dec = math.exp(d * float(prm.A[h]))
            for p in range(P):
                acc = 0.0
                for n in range(N):
                    s = float(Sw[i, h, p, n]) * dec + d * Bp[n] * float(x[i, h, p])
                    assert abs(s - float(S[i, h, p, n])) < 1e-12
                    acc += s * Cp[n]
                want = acc + float(prm.D[h]) * float(x[i, h, p])
                assert abs(want - float(y[i, h, p])) < 1e-10


def test_fresh_step_rotation_invariance():
    """Orthogonal R: B' = R B, C' = R C with S' = S R^T leaves y unchanged and keeps S' = S R^T
    (the per-head scalar decay commutes with R)."""
    gen, prm_r, S0 = _small(seed=7, b=2, H=8, P=16, G=2)
    prm_i = oracle.LayerParams(prm_r.H, prm_r.P, prm_r.N, prm_r.G, prm_r.dt_bias, prm_r.A, prm_r.D, None)
    f64 = torch.float64
    Rh = prm_r.R.double().repeat_interleave(8 // 2, dim=0)  # [H, N, N]: head h uses R of group h // HG
    S_plain = S0.double().clone()
    S_rot = torch.einsum("bhpn,hmn->bhpm", S_plain, Rh)  # S' = S R^T
    for _ in range(5):
        x, B, C, dt = oracle.make_step_inputs(2, 8, 16, N, 2, gen)
        y_plain = oracle.fresh_step(S_plain, x, B, C, dt, prm_i.to(f64), dtype=f64)
        y_rot = oracle.fresh_step(S_rot, x, B, C, dt, prm_r.to(f64), dtype=f64)
        assert torch.allclose(y_plain, y_rot, atol=1e-10)
    assert torch.allclose(S_rot, torch.einsum("bhpn,hmn->bhpm", S_plain, Rh), atol=1e-10)


# --------------------------------------------------------------------------- v4 native
def _fresh_traj(S0, steps_inputs, prm):
    """fp64 fresh trajectory: states S_t (after token t) and log decays a_t."""
    S = S0.double().clone()
    prm64 = prm.to(torch.float64)
    traj, ays = [S.clone()], []
    for (x, B, C, dt) in steps_inputs:
        oracle.fresh_step(S, x, B, C, dt, prm64, dtype=torch.float64)
        traj.append(S.clone())
        ays.append(oracle.softplus_dt(dt.double(), prm64.dt_bias) * prm64.A[None, :])
    return traj, ays


@pytest.mark.parametrize("k,c", [(32, 4), (64, 3), (96, 1), (32, 5)])
def test_native_v4_equals_stale_readout_closed_form(k, c):
    """y_t = S_t[:, :k] C'_t[:k] + exp(sum_{s=t0+1}^{t-1} a_s) S_{t0}[:, k:] C'_t[k:] + D x_t
    with t0 = c * floor((t-1)/c) the last snapshot: the one-token-lagged decay of
    scale/v4_native_decode.py:159-167. An inclusive decay or a wrong snapshot time fails."""
    b, H, P, G = 2, 4, 8, 2
    gen, prm, S0 = _small(seed=10 + k + c, b=b, H=H, P=P, G=G)
    steps = 3 * c + 2
    ins = [oracle.make_step_inputs(b, H, P, N, G, gen) for _ in range(steps)]
    traj, ays = _fresh_traj(S0, ins, prm)
    nat = oracle.NativeV4(b, H, P, N, k, c, dtype=torch.float64)
    nat.join(torch.arange(b), S0.double())
    prm64 = prm.to(torch.float64)
    for t in range(1, steps + 1):
        x, B, C, dt = ins[t - 1]
        y = nat.step(x, B, C, dt, prm)
        t0 = c * ((t - 1) // c)
        lag = sum((ays[s - 1] for s in range(t0 + 1, t)), torch.zeros(b, H, dtype=torch.float64))
        Cp = _heads(oracle.rotate(C.double(), prm64.R), H)
        want = torch.einsum("bhpn,bhn->bhp", traj[t][..., :k], Cp[..., :k]) + \
            torch.exp(lag)[..., None] * torch.einsum("bhpn,bhn->bhp", traj[t0][..., k:], Cp[..., k:]) + \
            x.double() * prm64.D[None, :, None]
        assert torch.allclose(y, want, atol=1e-11), f"t={t}"
        if t % c == 0:  # the snapshot after a flush is the fresh cold state
            assert torch.allclose(nat.snap, traj[t][..., k:], atol=1e-12)


def test_native_v4_all_hot_equals_fresh():
    """k = N reproduces fresh exactly (scale/v4_native_decode.py:16,77-78)."""
    b, H, P, G = 2, 8, 16, 2
    gen, prm, S0 = _small(seed=12, b=b, H=H, P=P, G=G)
    nat = oracle.NativeV4(b, H, P, N, N, 4)
    nat.join(torch.arange(b), S0)
    S = S0.clone()
    for _ in range(7):
        x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
        assert torch.equal(nat.step(x, B, C, dt, prm), oracle.fresh_step(S, x, B, C, dt, prm))


def test_native_v4_dt_min_path():
    b, H, P, G = 1, 4, 8, 1
    gen, prm, S0 = _small(seed=13, b=b, H=H, P=P, G=G, dt_min=0.2)
    nat = oracle.NativeV4(b, H, P, N, N, 4)
    nat.join(torch.arange(b), S0)
    S = S0.clone()
    x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
    y = nat.step(x, B, C, dt, prm)
    assert torch.equal(y, oracle.fresh_step(S, x, B, C, dt, prm))
    d = oracle.softplus_dt(dt.float(), prm.dt_bias, 0.2)
    assert float(d.min()) >= 0.2


@pytest.mark.parametrize("k,c", [(32, 4), (96, 1), (64, 7)])
def test_native_v4_exact_readout_equals_fresh_readout(k, c):
    """The rank-c exact correction (corr=1, scale/v4_native_decode.py:81-117) reads
    exp(G_t) snap + the buffered rank-1 terms, which is the current cold state: its y
    equals the fresh trajectory's y in fp64, with ragged phases and join/leave. The
    stale readout (the lagged decay, no correction) is checked to fail the same test,
    and so is a buffer that misses this token's term."""
    b, H, P, G = 3, 4, 8, 2
    gen, prm, S0 = _small(seed=40 + k + c, b=b, H=H, P=P, G=G)
    f64 = torch.float64
    prm64 = prm.to(f64)
    phase = torch.tensor([0, c // 2, c - 1])
    ex = oracle.NativeV4(b, H, P, N, k, c, dtype=f64, exact=True)
    st = oracle.NativeV4(b, H, P, N, k, c, dtype=f64)
    for m in (ex, st):
        m.join(torch.arange(b), S0.double(), phase)
    S = S0.double().clone()
    stale_differs = False
    for step in range(3 * c + 5):
        if step == c + 1:  # slot 1 leaves, a new request joins it mid-window
            Sj = oracle.make_state(1, H, P, N, gen).double()
            S[1] = Sj[0]
            for m in (ex, st):
                m.join(torch.tensor([1]), Sj, torch.tensor([1 % c]))
        x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
        y_fresh = oracle.fresh_step(S, x, B, C, dt, prm64, dtype=f64)
        y_ex = ex.step(x, B, C, dt, prm)
        y_st = st.step(x, B, C, dt, prm)
        assert torch.allclose(y_ex, y_fresh, atol=1e-11), f"step {step}"
        stale_differs |= not torch.allclose(y_st, y_fresh, atol=1e-6)
        # without this token's term (dt x)_t (C'_cold . B'_t) the readout is off
        xf, Bp, Cp, dtv, a = oracle.v4_ref._prep(x, B, C, dt, prm64, f64)
        own = dtv[..., None] * xf * torch.einsum("bhn,bhn->bh", Bp[..., k:], Cp[..., k:])[..., None]
        assert not torch.allclose(y_ex - own, y_fresh, atol=1e-6)
    assert stale_differs


def test_native_v4_exact_fp8_is_fresh_plus_snapshot_quantisation():
    """exact readout with an e4m3 snapshot = fresh readout + exp(G_t) ((q sc - snap) . C'_cold),
    the snapshot being the fresh cold state at the last flush (one quantisation, no re-store)."""
    b, H, P, G, k, c = 2, 4, 8, 2, 32, 4
    gen, prm, S0 = _small(seed=47, b=b, H=H, P=P, G=G)
    f64 = torch.float64
    prm64 = prm.to(f64)
    ex = oracle.NativeV4(b, H, P, N, k, c, cold="fp8", dtype=f64, fp8_restore_each_step=False, exact=True)
    ex.join(torch.arange(b), S0.double())
    S = S0.double().clone()
    snap = S[..., k:].clone()
    G_t = torch.zeros(b, H, dtype=f64)
    for t in range(1, 3 * c + 2):
        x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
        q, sc = oracle.quant_fp8(snap.float())
        err = oracle.read_fp8(q, sc).double() - snap
        xf, Bp, Cp, dtv, a = oracle.v4_ref._prep(x, B, C, dt, prm64, f64)
        G_t = G_t + a
        y_fresh = oracle.fresh_step(S, x, B, C, dt, prm64, dtype=f64)
        want = y_fresh + torch.exp(G_t)[..., None] * torch.einsum("bhpn,bhn->bhp", err, Cp[..., k:])
        assert torch.allclose(ex.step(x, B, C, dt, prm), want, atol=1e-10), f"t={t}"
        if t % c == 0:
            snap = S[..., k:].clone()
            G_t = torch.zeros_like(G_t)


# --------------------------------------------------------------------------- tiered
def test_tiered_chunked_replay_equals_native_recurrence_ragged():
    """The chunked flush (scale/v4_fused_decode.py:76-85) equals the per-token
    recurrence in fp64, with per-slot phases, partial batches and join/leave."""
    slots, H, P, G, k, c = 5, 4, 8, 2, 32, 4
    gen, prm, S0 = _small(seed=14, b=slots, H=H, P=P, G=G)
    phase = torch.tensor([0, 1, 2, 3, 2])
    f64 = torch.float64
    nat = oracle.NativeV4(slots, H, P, N, k, c, dtype=f64)
    tie = oracle.TieredV4(slots, H, P, N, G, k, c, dtype=f64)
    nat.join(torch.arange(slots), S0.double(), phase)
    tie.join(torch.arange(slots), S0.double(), phase)
    for step in range(30):
        if step == 13:
            Sj = oracle.make_state(1, H, P, N, gen).double()
            nat.join(torch.tensor([2]), Sj, torch.tensor([3]))
            tie.join(torch.tensor([2]), Sj, torch.tensor([3]))
        sl = torch.randperm(slots, generator=gen)[:3 + step % 3]
        x, B, C, dt = oracle.make_step_inputs(len(sl), H, P, N, G, gen)
        y1 = nat.step(x, B, C, dt, prm, slots=sl)
        y2 = tie.step(x, B, C, dt, prm, slots=sl)
        assert torch.allclose(y1, y2, atol=1e-12)
    assert torch.allclose(tie.materialize(torch.arange(slots), prm), nat.S, atol=1e-12)


def test_tiered_flush_weights_detect_a_dropped_decay_term():
    """A replay that forgets the suffix decay of older tokens disagrees with the
    recurrence: the closed form is not retyped, it is checked against it."""
    f64 = torch.float64
    slots, H, P, G, k, c = 1, 2, 4, 1, 32, 4
    gen, prm, S0 = _small(seed=15, b=slots, H=H, P=P, G=G)
    tie = oracle.TieredV4(slots, H, P, N, G, k, c, dtype=f64)
    tie.join(torch.arange(1), S0.double())
    nat = oracle.NativeV4(slots, H, P, N, k, c, dtype=f64)
    nat.join(torch.arange(1), S0.double())
    for _ in range(c - 1):
        ins = oracle.make_step_inputs(1, H, P, N, G, gen)
        tie.step(*ins, prm)
        nat.step(*ins, prm)
    entries = tie.ring[0]
    broken = [(e[0], e[1], e[2]) for e in entries]
    dts = torch.stack([e[0] for e in broken])
    X = torch.stack([e[1] for e in broken])
    Bc = torch.stack([e[2] for e in broken])
    a = dts * prm.to(f64).A[None, :]
    no_suffix = tie.cold[0] * torch.exp(a.sum(0))[:, None, None] + torch.einsum("mh,mhp,mhn->hpn", dts, X, Bc)
    good = tie.materialize(torch.arange(1), prm)[0][..., k:]
    assert torch.allclose(good, nat.S[0][..., k:], atol=1e-12)
    assert not torch.allclose(no_suffix, nat.S[0][..., k:], atol=1e-6)


# --------------------------------------------------------------------------- fp8 / bf16
def test_quant_fp8_row_scale_and_error_bound():
    gen = torch.Generator().manual_seed(16)
    s = torch.randn(3, 5, 96, generator=gen) * torch.logspace(-4, 1, 5)[None, :, None]
    q, sc = oracle.quant_fp8(s)
    assert q.dtype == torch.float8_e4m3fn and sc.shape == (3, 5, 1)
    amax = s.abs().amax(-1, keepdim=True)
    assert torch.equal(sc, amax / 448.0 + 1e-12)
    d = oracle.read_fp8(q, sc)
    # the row maximum lands on the largest finite code; every element within half an e4m3 ulp
    assert torch.allclose(d.abs().amax(-1, keepdim=True), amax, rtol=2 ** -4)
    rel = ((d - s).abs() / s.abs().clamp_min(sc * 2 ** -6)).max()
    assert float(rel) <= 2 ** -4 + 1e-6


def test_native_v4_fp8_tracks_fp32_within_quantisation_error():
    b, H, P, G, k, c = 2, 8, 16, 2, 32, 4
    gen, prm, S0 = _small(seed=17, b=b, H=H, P=P, G=G)
    n32 = oracle.NativeV4(b, H, P, N, k, c, cold="fp32")
    n8 = oracle.NativeV4(b, H, P, N, k, c, cold="fp8")
    n8b = oracle.NativeV4(b, H, P, N, k, c, cold="fp8", fp8_restore_each_step=False)
    for n in (n32, n8, n8b):
        n.join(torch.arange(b), S0)
    for _ in range(12):
        x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
        y32 = n32.step(x, B, C, dt, prm)
        y8 = n8.step(x, B, C, dt, prm)
        y8b = n8b.step(x, B, C, dt, prm)
        rel = float((y8 - y32).norm() / y32.norm())
        assert 0 < rel < 2e-2
        # re-storing the dequantized snapshot each step (scale/vllm_v4_patch.py:173-175)
        # keeps every code; only the row scale drifts (~1e-8 relative per re-store,
        # from the +1e-12 term), so it matches quantizing at the flush only
        assert torch.equal(n8.q8.view(torch.uint8), n8b.q8.view(torch.uint8))
        assert float((n8.sc8 - n8b.sc8).abs().max() / n8b.sc8.abs().max()) < 1e-6
        assert float((y8 - y8b).norm() / y8b.norm()) < 1e-7


def test_native_v4_bf16_snapshot_is_rne_of_fp32():
    b, H, P, G, k, c = 1, 4, 8, 1, 32, 2
    gen, prm, S0 = _small(seed=18, b=b, H=H, P=P, G=G)
    nb = oracle.NativeV4(b, H, P, N, k, c, cold="bf16")
    nb.join(torch.arange(b), S0)
    for _ in range(4):
        nb.step(*oracle.make_step_inputs(b, H, P, N, G, gen), prm)
    assert torch.equal(nb.snap, nb.S[..., k:].to(torch.bfloat16).float())


def test_native_v4_hot_only_and_qgate_readouts():
    """coldoff=1 (hot-only draft readout) and the query-gated cold skip, against an fp64
    restatement built from the stale readout and the hot columns of a fresh trajectory:
    hot_only y = hot C'[:k] + D x; qgate y = stale y for kept heads, hot-only y for the
    others, keep computed from the rotated C of each group (a head inherits its group's C');
    tau = 0 is the stale readout, tau above 1 the hot-only one; the state evolves as in the
    stale readout either way."""
    b, H, P, G, k, c = 3, 8, 16, 2, 32, 4
    gen, prm, S0 = _small(seed=43, b=b, H=H, P=P, G=G)
    f64 = torch.float64
    stale = oracle.NativeV4(b, H, P, N, k, c, dtype=f64)
    gated = oracle.NativeV4(b, H, P, N, k, c, dtype=f64)
    hot = oracle.NativeV4(b, H, P, N, k, c, dtype=f64)
    for n in (stale, gated, hot):
        n.join(torch.arange(b), S0.double())
    S = S0.double().clone()
    prm64 = prm.to(f64)
    tau = 0.75  # the cold fraction of |C'|^2 is about 96/128 for random C: about half the heads kept
    kept_total = 0
    for step in range(2 * c + 1):
        x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
        y_s = stale.step(x, B, C, dt, prm)
        y_g = gated.step(x, B, C, dt, prm, qgate=tau)
        y_h = hot.step(x, B, C, dt, prm, hot_only=True)
        oracle.fresh_step(S, x, B, C, dt, prm64, dtype=f64)
        Cp = _heads(oracle.rotate(C.double(), prm64.R), H)
        y_hot_ref = torch.einsum("bhpn,bhn->bhp", S[..., :k], Cp[..., :k]) + x.double() * prm64.D[None, :, None]
        assert torch.allclose(y_h, y_hot_ref, atol=1e-12)
        rho = (Cp[..., k:] ** 2).sum(-1) / (Cp ** 2).sum(-1)
        keep = rho >= tau
        kept_total += int(keep.sum())
        assert 0 < int(keep.sum()) < keep.numel()
        want = torch.where(keep[..., None], y_s, y_h)
        assert torch.allclose(y_g, want, atol=1e-12)
    assert gated.qgate_n == (2 * c + 1) * b * H and gated.qgate_kept == kept_total
    # the bookkeeping runs as in the stale readout
    for n in (gated, hot):
        assert torch.equal(n.S, stale.S) and torch.equal(n.snap, stale.snap) and torch.equal(n.glog, stale.glog)
    # tau = 0 is the stale readout; tau above 1 the hot-only one
    a0, a1, a2, a3 = (oracle.NativeV4(b, H, P, N, k, c, dtype=f64) for _ in range(4))
    for n in (a0, a1, a2, a3):
        n.join(torch.arange(b), S0.double())
    ins = oracle.make_step_inputs(b, H, P, N, G, gen)
    assert torch.equal(a0.step(*ins, prm, qgate=0.0), a1.step(*ins, prm))
    assert torch.equal(a2.step(*ins, prm, qgate=1.5), a3.step(*ins, prm, hot_only=True))
    # a query whose rotated C' lies in one cold column (C = R^T e_n, n >= k) has rho = 1 and
    # is kept for tau = 0.95; one in a hot column (n < k) has rho ~ 0 and is dropped for
    # tau = 0.05 (a swapped fraction or a transposed R fails this)
    for col, tau_, kept in ((k + 7, 0.95, True), (3, 0.05, False)):
        Cq = torch.zeros(b, G, N, dtype=f64)
        Cq[..., col] = 1.0
        Cq = torch.einsum("gmn,bgm->bgn", prm64.R, Cq).to(torch.bfloat16)  # R^T e_col per group
        n_ = oracle.NativeV4(b, H, P, N, k, c, dtype=f64)
        n_.join(torch.arange(b), S0.double())
        n_.step(ins[0], ins[1], Cq, ins[3], prm, qgate=tau_)
        assert n_.qgate_kept == (b * H if kept else 0)


def _bf16(v: torch.Tensor) -> torch.Tensor:
    return v.to(torch.bfloat16).to(v.dtype)


@pytest.mark.parametrize("cold", ["bf16", "fp8"])
def test_native_v4_bf16_master_is_fresh_recurrence_rounded_at_each_flush(cold):
    """master="bf16" (the fused path's bf16 master, scale/v4_fused_decode.py:149,156-158)
    against a brute-force restatement built from fresh_step in fp64: the state is the
    fresh recurrence whose cold columns are rounded to bf16 at the join and after every
    flush token, and the read copy comes from those rounded values (bf16: the same
    values, a single copy; e4m3: quant_fp8 of them). Rounding at every token, never, or
    quantizing the unrounded state each fails one of the checks."""
    b, H, P, G, k, c = 2, 8, 16, 2, 32, 4
    gen, prm, S0 = _small(seed=41, b=b, H=H, P=P, G=G)
    f64 = torch.float64
    nat = oracle.NativeV4(b, H, P, N, k, c, cold=cold, dtype=f64, master="bf16")
    exact = oracle.NativeV4(b, H, P, N, k, c, cold=cold, dtype=f64)  # fp32 (unrounded) master
    nat.join(torch.arange(b), S0.double())
    exact.join(torch.arange(b), S0.double())
    S = S0.double().clone()
    S[..., k:] = _bf16(S[..., k:])
    every = S.clone()  # rounded at every token: a plausible mistake
    prm64 = prm.to(f64)
    for step in range(3 * c):
        ins = oracle.make_step_inputs(b, H, P, N, G, gen)
        nat.step(*ins, prm)
        exact.step(*ins, prm)
        oracle.fresh_step(S, *ins, prm64, dtype=f64)
        oracle.fresh_step(every, *ins, prm64, dtype=f64)
        every[..., k:] = _bf16(every[..., k:])
        if (step + 1) % c == 0:
            S[..., k:] = _bf16(S[..., k:])
            if cold == "bf16":  # single copy: the read copy is the master
                assert torch.equal(nat.snap, S[..., k:])
            else:
                q, sc = oracle.quant_fp8(S[..., k:].float())
                assert torch.equal(nat.q8.view(torch.uint8), q.view(torch.uint8))
                assert torch.equal(nat.sc8, sc)
                q_unrounded, _ = oracle.quant_fp8(exact.S[..., k:].float())
                assert not torch.equal(q.view(torch.uint8), q_unrounded.view(torch.uint8))
        assert torch.allclose(nat.S, S, rtol=0, atol=1e-12)
    assert not torch.allclose(every, S, rtol=0, atol=1e-6)
    assert not torch.allclose(exact.S, S, rtol=0, atol=1e-6)


def test_tiered_bf16_master_equals_native_bf16_master_ragged():
    """The chunked replay into a bf16 master (round the replayed window once) equals
    the per-token recurrence rounded at the flush, in fp64, with per-slot phases,
    partial batches and join/leave."""
    slots, H, P, G, k, c = 5, 4, 8, 2, 32, 4
    gen, prm, S0 = _small(seed=42, b=slots, H=H, P=P, G=G)
    phase = torch.tensor([0, 1, 2, 3, 2])
    f64 = torch.float64
    nat = oracle.NativeV4(slots, H, P, N, k, c, cold="bf16", dtype=f64, master="bf16")
    tie = oracle.TieredV4(slots, H, P, N, G, k, c, dtype=f64, master="bf16")
    nat.join(torch.arange(slots), S0.double(), phase)
    tie.join(torch.arange(slots), S0.double(), phase)
    for step in range(30):
        if step == 13:
            Sj = oracle.make_state(1, H, P, N, gen).double()
            nat.join(torch.tensor([2]), Sj, torch.tensor([3]))
            tie.join(torch.tensor([2]), Sj, torch.tensor([3]))
        sl = torch.randperm(slots, generator=gen)[:3 + step % 3]
        x, B, C, dt = oracle.make_step_inputs(len(sl), H, P, N, G, gen)
        y1 = nat.step(x, B, C, dt, prm, slots=sl)
        y2 = tie.step(x, B, C, dt, prm, slots=sl)
        assert torch.allclose(y1, y2, atol=1e-12)
    assert torch.allclose(tie.materialize(torch.arange(slots), prm), nat.S, atol=1e-12)


def test_fp8_readout_matches_fp64_loop():
    gen = torch.Generator().manual_seed(19)
    R_, Nc, Pd = 3, 6, 5
    q = torch.randn(R_, Nc, generator=gen)
    sc = torch.rand(R_, Nc, generator=gen) + 0.1
    S8 = torch.randn(R_, Nc, Pd, generator=gen).to(torch.float8_e4m3fn)
    got = oracle.fp8_readout(q, S8, sc)
    for r in range(R_):
        for p in range(Pd):
            want = sum(float(q[r, n]) * float(sc[r, n]) * float(S8[r, n, p].float()) for n in range(Nc))
            assert abs(want - float(got[r, p])) < 1e-5


def test_hot_only_step_is_the_fresh_trajectory_restricted_to_hot_columns():
    b, H, P, G, k = 2, 4, 8, 2, 32
    gen, prm, S0 = _small(seed=20, b=b, H=H, P=P, G=G)
    ins = [oracle.make_step_inputs(b, H, P, N, G, gen) for _ in range(5)]
    traj, _ = _fresh_traj(S0, ins, prm)
    Sh = S0[..., :k].double().clone()
    prm64 = prm.to(torch.float64)
    for t, (x, B, C, dt) in enumerate(ins, start=1):
        y = oracle.hot_only_step(Sh, x, B, C, dt, prm64, dtype=torch.float64)
        Cp = _heads(oracle.rotate(C.double(), prm64.R), H)
        want = torch.einsum("bhpn,bhn->bhp", traj[t][..., :k], Cp[..., :k]) + x.double() * prm64.D[None, :, None]
        assert torch.allclose(y, want, atol=1e-11)
        assert torch.allclose(Sh, traj[t][..., :k], atol=1e-12)


# --------------------------------------------------------------------------- conv prologue
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_conv_update_matches_transformers_causal_conv1d_update(dtype):
    """The conv prologue against transformers' causal_conv1d_update (the installed
    library's restatement of causal-conv1d's kernel) with SiLU, in the model dtype;
    the state update is bit-exact, the outputs agree to the bf16 cast."""
    from transformers.models.nemotron_h import modeling_nemotron_h as M

    gen = torch.Generator().manual_seed(50)
    b, I, gn, W = 3, 40, 16, 4
    dim = I + 2 * gn
    hbc = torch.randn(b, dim, generator=gen).to(dtype)
    st = torch.randn(b, dim, W, generator=gen).to(dtype)
    w = (torch.randn(dim, W, generator=gen) * 0.5).to(dtype)
    bias = torch.randn(dim, generator=gen).to(dtype)
    st_ref = st.clone()
    out = M.causal_conv1d_update(hbc[..., None], st_ref, w, bias, activation="silu")[..., 0]
    st_me = st.clone()
    x, B, C = oracle.conv_update(hbc, st_me, w, bias, I, gn)
    assert torch.equal(st_me, st_ref)
    got = torch.cat([x, B, C], dim=-1).float()
    want = out.to(torch.bfloat16).float()
    assert torch.allclose(got, want, rtol=2 ** -7, atol=1e-6)
    assert float((got != want).float().mean()) < 0.02


def test_conv_update_matches_fp64_window_loop():
    gen = torch.Generator().manual_seed(51)
    b, I, gn, W = 2, 8, 4, 3
    dim = I + 2 * gn
    hbc = torch.randn(b, dim, generator=gen)
    st = torch.randn(b, dim, W, generator=gen)
    w = torch.randn(dim, W, generator=gen)
    bias = torch.randn(dim, generator=gen)
    mask = torch.tensor([1.0, 0.0])
    want = torch.zeros(b, dim, dtype=torch.float64)
    for r in range(b):
        for ch in range(dim):
            win = [float(st[r, ch, k]) for k in range(1, W)] + [float(hbc[r, ch])]
            v = float(bias[ch]) + sum(win[k] * float(w[ch, k]) for k in range(W))
            want[r, ch] = v / (1.0 + math.exp(-v)) * float(mask[r])
    x, B, C = oracle.conv_update(hbc, st.clone(), w, bias, I, gn, mask=mask)
    got = torch.cat([x, B, C], dim=-1).double()
    assert torch.allclose(got, want.to(torch.bfloat16).double(), rtol=2 ** -7, atol=1e-6)


# --------------------------------------------------------------------------- epilogue
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_rmsnorm_matches_transformers_module(dtype):
    from transformers.models.nemotron_h import modeling_nemotron_h as M

    gen = torch.Generator().manual_seed(60)
    b, I, gs = 3, 96, 32
    norm = M.Zamba2RMSNormGated(I, group_size=gs, eps=1e-5).to(dtype)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(I, generator=gen).to(dtype))
    y = torch.randn(b, I, generator=gen)
    gate = torch.randn(b, I, generator=gen).to(dtype)
    with torch.no_grad():
        want = norm(y.to(dtype), gate)
    got = oracle.gated_rmsnorm(y, gate, norm.weight.detach(), gs, 1e-5)
    assert got.dtype == want.dtype
    assert torch.equal(got, want)


def test_gated_rmsnorm_matches_fp64_group_loop():
    gen = torch.Generator().manual_seed(61)
    b, I, gs = 2, 12, 4
    y, gate, w = torch.randn(b, I, generator=gen), torch.randn(b, I, generator=gen), torch.randn(I, generator=gen)
    want = torch.zeros(b, I, dtype=torch.float64)
    for r in range(b):
        for g0 in range(0, I, gs):
            v = [float(y[r, i]) * float(gate[r, i]) / (1 + math.exp(-float(gate[r, i]))) for i in range(g0, g0 + gs)]
            rs = 1 / math.sqrt(sum(t * t for t in v) / gs + 1e-6)
            for j, i in enumerate(range(g0, g0 + gs)):
                want[r, i] = float(w[i]) * v[j] * rs
    got = oracle.gated_rmsnorm(y, gate, w, gs, 1e-6)
    assert torch.allclose(got.double(), want, rtol=1e-6, atol=1e-7)


# --------------------------------------------------------------------------- teacher-forced v4
@pytest.mark.parametrize("k,c", [(32, 4), (16, 3), (96, 1), (32, 5), (0, 4), (0, 1)])
def test_teacher_forced_v4_equals_closed_form(k, c):
    """scale/nemo9b_eval.py:41-85 (mode "v4"; k = 0 is mode "c1", :79-80): at sequence position tau,
    y = S_tau[:k] C'[:k] + exp(sum_{i=ts+1}^{tau} a_i) S_ts[k:] C'[k:] + D x with
    ts = c floor(tau / c) and S_ts the state AFTER token ts's update (fp64 fresh trajectory).
    Negative controls: an exclusive decay (sum to tau - 1) and a snapshot taken before the
    update (S_{ts-1}) both miss."""
    b, H, P, G = 2, 4, 8, 2
    gen, prm, S0 = _small(seed=300 + k + c, b=b, H=H, P=P, G=G)
    steps = 3 * c + 2
    ins = [oracle.make_step_inputs(b, H, P, N, G, gen) for _ in range(steps)]
    traj, ays = _fresh_traj(S0, ins, prm)  # traj[i + 1]: after token i; ays[i]: token i's log decay
    tf = oracle.TeacherForcedV4(b, H, P, N, k, c, dtype=torch.float64)
    tf.join(torch.arange(b), S0.double())
    prm64 = prm.to(torch.float64)
    zero = torch.zeros(b, H, dtype=torch.float64)
    for tau in range(steps):
        x, B, C, dt = ins[tau]
        y = tf.step(x, B, C, dt, prm)
        ts = c * (tau // c)
        Cp = _heads(oracle.rotate(C.double(), prm64.R), H)
        dx = x.double() * prm64.D[None, :, None]
        hot = torch.einsum("bhpn,bhn->bhp", traj[tau + 1][..., :k], Cp[..., :k])

        def cold(state, lag):
            return torch.exp(lag)[..., None] * torch.einsum("bhpn,bhn->bhp", state[..., k:], Cp[..., k:])

        inc = sum((ays[i] for i in range(ts + 1, tau + 1)), zero)
        want = hot + cold(traj[ts + 1], inc) + dx
        assert torch.allclose(y, want, atol=1e-11), f"tau={tau}"
        if tau > ts:
            exc = sum((ays[i] for i in range(ts + 1, tau)), zero)
            assert float((y - (hot + cold(traj[ts + 1], exc) + dx)).abs().max()) > 1e-6
        assert float((y - (hot + cold(traj[ts], inc) + dx)).abs().max()) > 1e-6


@pytest.mark.parametrize("k,c", [(32, 4), (16, 3), (0, 4), (32, 1)])
def test_teacher_forced_v4_lagged_equals_closed_form(k, c):
    """scale/nemo9b_eval.py:44,59,70 (lag = 1, the asynchronous-flush model): readers see the
    snapshot before the last one. At position tau the cold term is
    exp(sum_{i=lo}^{tau} a_i) S_lo[k:] C'[k:] with lo = c (floor(tau / c) - 1) + 1 (the state
    after token c (floor(tau / c) - 1)), or lo = 0 (the joined state) for tau < c. Negative
    control: the unlagged snapshot (lo = c floor(tau / c) + 1) misses from the second window on."""
    b, H, P, G = 2, 4, 8, 2
    gen, prm, S0 = _small(seed=330 + k + c, b=b, H=H, P=P, G=G)
    steps = 3 * c + 2
    ins = [oracle.make_step_inputs(b, H, P, N, G, gen) for _ in range(steps)]
    traj, ays = _fresh_traj(S0, ins, prm)
    tf = oracle.TeacherForcedV4(b, H, P, N, k, c, dtype=torch.float64, lag=1)
    tf.join(torch.arange(b), S0.double())
    prm64 = prm.to(torch.float64)
    zero = torch.zeros(b, H, dtype=torch.float64)
    for tau in range(steps):
        x, B, C, dt = ins[tau]
        y = tf.step(x, B, C, dt, prm)
        Cp = _heads(oracle.rotate(C.double(), prm64.R), H)
        dx = x.double() * prm64.D[None, :, None]
        hot = torch.einsum("bhpn,bhn->bhp", traj[tau + 1][..., :k], Cp[..., :k])

        def term(lo):
            dec = sum((ays[i] for i in range(lo, tau + 1)), zero)
            return torch.exp(dec)[..., None] * torch.einsum("bhpn,bhn->bhp", traj[lo][..., k:], Cp[..., k:])

        lo = c * (tau // c - 1) + 1 if tau >= c else 0
        assert torch.allclose(y, hot + term(lo) + dx, atol=1e-11), f"tau={tau}"
        if tau >= c:
            assert float((y - (hot + term(c * (tau // c) + 1) + dx)).abs().max()) > 1e-6


def test_teacher_forced_v4_reduces_to_fresh_and_differs_from_decode():
    """c = 1 (a snapshot after every update) and k = N give the fresh readout; warm tokens
    read fresh; the decode readout (NativeV4, one-token-lagged snapshot) is another one."""
    b, H, P, G = 2, 8, 16, 2
    gen, prm, S0 = _small(seed=320, b=b, H=H, P=P, G=G)
    ins = [oracle.make_step_inputs(b, H, P, N, G, gen) for _ in range(9)]
    fresh_S = S0.clone()
    arms = {"c1": oracle.TeacherForcedV4(b, H, P, N, 32, 1), "kN": oracle.TeacherForcedV4(b, H, P, N, N, 4),
            "warm": oracle.TeacherForcedV4(b, H, P, N, 32, 4, warm=3),
            "tf": oracle.TeacherForcedV4(b, H, P, N, 32, 4)}
    for a in arms.values():
        a.join(torch.arange(b), S0)
    dec = oracle.NativeV4(b, H, P, N, 32, 4)
    dec.join(torch.arange(b), S0)
    gap = 0.0
    for tau, (x, B, C, dt) in enumerate(ins):
        yf = oracle.fresh_step(fresh_S, x, B, C, dt, prm)
        ys = {n: a.step(x, B, C, dt, prm) for n, a in arms.items()}
        yd = dec.step(x, B, C, dt, prm)
        assert torch.allclose(ys["c1"], yf, atol=1e-6)
        assert torch.allclose(ys["kN"], yf, atol=1e-6)
        if tau < 3 or tau % 4 == 0:  # warm tokens read the fresh state, and so do snapshot tokens
            assert torch.allclose(ys["warm"], yf, atol=1e-6)
        if tau % 4 == 0:
            assert torch.allclose(ys["tf"], yf, atol=1e-6)
        gap = max(gap, float((ys["tf"] - yd).abs().max()))
    assert gap > 1e-3


def test_teacher_forced_v4_fp8_row_scale_is_close_to_the_column_scale():
    """The reference's evaluation scales its e4m3 snapshot per column (amax over P,
    scale/nemo9b_eval.py:62-64); the tier's format scales per row (amax over the cold
    columns). Both stay within the 2e-2 fp8 bar of the fp32 snapshot and of each other."""
    b, H, P, G, k, c = 2, 8, 80, 2, 32, 4
    gen, prm, S0 = _small(seed=330, b=b, H=H, P=P, G=G)
    arms = {n: oracle.TeacherForcedV4(b, H, P, N, k, c, cold=cold, fp8_scale=sc)
            for n, cold, sc in (("fp32", "fp32", "row"), ("row", "fp8", "row"), ("col", "fp8", "column"))}
    for a in arms.values():
        a.join(torch.arange(b), S0)
    for _ in range(2 * c + 1):
        x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
        ys = {n: a.step(x, B, C, dt, prm) for n, a in arms.items()}
        rel = lambda u, v: float((u - v).norm() / v.norm())  # noqa: E731
        assert rel(ys["row"], ys["fp32"]) <= 2e-2 and rel(ys["col"], ys["fp32"]) <= 2e-2
        assert rel(ys["row"], ys["col"]) <= 2e-2


@pytest.mark.parametrize("cold,k,c", [("bf16", 32, 4), ("fp8", 32, 3), ("fp8", 0, 4), ("bf16", 16, 1)])
def test_teacher_forced_v4_bf16_master_state_is_the_rounded_recurrence(cold, k, c):
    """master="bf16": the state is the fp64 fresh recurrence with the cold columns rounded to
    bf16 at the join and at every snapshot position (t % c == 0) - the state NativeV4's pinned
    bf16 master holds when its flushes fall on the same tokens (joined at phase c - 1) - and
    the snapshot is the quantization of the rounded values. Negative controls: without the
    rounding, and with a rounding at every token, the state differs."""
    b, H, P, G = 2, 4, 16, 2
    gen, prm, S0 = _small(seed=340 + k + c, b=b, H=H, P=P, G=G)
    S0 = S0 * 7.0  # magnitudes whose bf16 rounding is far above fp64 noise
    tf = oracle.TeacherForcedV4(b, H, P, N, k, c, cold=cold, master="bf16", dtype=torch.float64)
    tf.join(torch.arange(b), S0.double())
    nat = oracle.NativeV4(b, H, P, N, k, c, cold=cold, master="bf16", dtype=torch.float64) if k else None
    if nat is not None:
        nat.join(torch.arange(b), S0.double(), phase=torch.full((b,), c - 1))
    rnd = lambda S: torch.cat([S[..., :k], S[..., k:].to(torch.bfloat16).double()], -1)  # noqa: E731
    S = rnd(S0.double())
    S_none, S_every = S0.double().clone(), rnd(S0.double())
    prm64 = prm.to(torch.float64)
    for tau in range(3 * c + 2):
        x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
        tf.step(x, B, C, dt, prm)
        for T in (S, S_none, S_every):
            oracle.fresh_step(T, x, B, C, dt, prm64, dtype=torch.float64)
        if tau % c == 0:
            S.copy_(rnd(S))
            snap = S[..., k:].clone()
        S_every.copy_(rnd(S_every))
        assert torch.allclose(tf.S, S, rtol=0, atol=1e-12), f"tau={tau}"
        if nat is not None:
            nat.step(x, B, C, dt, prm)
            assert torch.allclose(nat.S, S, rtol=0, atol=1e-12), f"NativeV4 tau={tau}"
        if tau > 0:
            assert float((tf.S - S_none).abs().max()) > 1e-7
        if tau % c != 0:
            assert float((tf.S - S_every).abs().max()) > 1e-7
    # the snapshot is the quantization of the rounded cold columns at the last snapshot token
    if cold == "bf16":
        assert torch.equal(tf.snap, snap.to(torch.bfloat16).double())
    else:
        assert torch.equal(tf.snap, oracle.read_fp8(*oracle.quant_fp8(snap.float())).double())


def test_mask_width_is_the_width_dimensional_model():
    """set_width (scale/nemotron_retrofit.py:29-37, :114-116): mask_width keeps the first w
    coordinates of an explicit fp64 rotation R B; a fresh trajectory under it keeps state
    columns >= w at exactly zero and equals the w-dimensional model built from the first w
    rows of R (S_w <- exp(a) S_w + dt x (R_w B), y = S_w (R_w C) + D x) - not the full
    model, and not the identity rotation masked."""
    b, H, P, G, w = 2, 4, 8, 2, 48
    gen, prm, _ = _small(seed=350, b=b, H=H, P=P, G=G)
    R = prm.R.double()
    X = torch.randn(5, G, N, generator=gen, dtype=torch.float64)
    want = torch.zeros(5, G, N, dtype=torch.float64)
    for t in range(5):
        for g in range(G):
            want[t, g, :w] = R[g, :w] @ X[t, g]
    assert torch.allclose(oracle.mask_width(oracle.rotate(X, R), w), want, atol=1e-12)
    S = torch.zeros(b, H, P, N, dtype=torch.float64)
    S_full = S.clone()
    Sw = torch.zeros(b, H, P, w, dtype=torch.float64)
    prm64 = prm.to(torch.float64)
    Rh = R[:, :w].repeat_interleave(H // G, dim=0)  # [H, w, N]
    for tau in range(6):
        x, B, C, dt = oracle.make_step_inputs(b, H, P, N, G, gen)
        y = oracle.fresh_step(S, x, B, C, dt, prm64, dtype=torch.float64, width=w)
        y_full = oracle.fresh_step(S_full, x, B, C, dt, prm64, dtype=torch.float64)
        d = oracle.softplus_dt(dt.double(), prm64.dt_bias)
        a = d * prm64.A[None, :]
        Bw = torch.einsum("hmn,bhn->bhm", Rh, B.double().repeat_interleave(H // G, dim=1))
        Cw = torch.einsum("hmn,bhn->bhm", Rh, C.double().repeat_interleave(H // G, dim=1))
        Sw = Sw * torch.exp(a)[..., None, None] + (d[..., None] * x.double())[..., None] * Bw[:, :, None, :]
        y_w = torch.einsum("bhpm,bhm->bhp", Sw, Cw) + x.double() * prm64.D[None, :, None]
        assert torch.equal(S[..., w:], torch.zeros_like(S[..., w:]))
        assert torch.allclose(S[..., :w], Sw, atol=1e-12) and torch.allclose(y, y_w, atol=1e-12)
        assert float((y - y_full).abs().max()) > 1e-4
