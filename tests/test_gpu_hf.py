"""GPU: the transformers drop-in modules (v4_native_decode / v4_fused_decode)
on a tiny random-init NemotronH (fp32 weights; the mixers hand bf16 x, B, C,
dt to the kernels as the 9B model does).

The adapters' state handling is checked against the oracle: every decode call
records the kernel inputs and the kernel's y, the prefill state the tier was
built from is recorded, and the oracle replays the same sequence (fp32 bar,
rtol = atol = 1e-5)."""
import pytest
import torch

import oracle
from helpers import assert_close32

pytestmark = pytest.mark.gpu

N = 128


def _tiny_model(seed=0, rotated=True):
    from transformers import NemotronHConfig, NemotronHForCausalLM

    from nested_ssm_amd import hf

    torch.manual_seed(seed)
    cfg = NemotronHConfig(vocab_size=96, hidden_size=128, layers_block_type=["mamba", "attention", "mamba"],
                          num_attention_heads=4, num_key_value_heads=2, head_dim=32, intermediate_size=256,
                          ssm_state_size=N, mamba_num_heads=8, mamba_head_dim=16, n_groups=2, conv_kernel=4,
                          chunk_size=16, use_mamba_kernels=False, attn_implementation="eager")
    model = NemotronHForCausalLM(cfg).to("cuda", torch.float32).eval()
    gen = torch.Generator().manual_seed(seed + 1)
    rgen = torch.Generator().manual_seed(seed + 2)  # R draws do not shift the other parameters
    for m in hf.mixers(model):
        with torch.no_grad():  # spread decays and skips so the test sees varied heads
            m.A_log.copy_(torch.rand(m.num_heads, generator=gen) * 2.7)
            m.dt_bias.copy_(torch.log(torch.expm1(0.001 + 0.099 * torch.rand(m.num_heads, generator=gen))))
            m.D.copy_(torch.randn(m.num_heads, generator=gen))
        if rotated:
            m.act = hf.ActRotMask(m.act, m.intermediate_size, m.n_groups, m.ssm_state_size).cuda()
            with torch.no_grad():
                m.act.R.copy_(oracle.make_rotation(m.n_groups, N, rgen))
    return model


class Recorder:
    """Wraps the adapter's capture / decode_inputs / decode_epilogue."""

    def __init__(self, monkeypatch):
        from nested_ssm_amd import hf

        self.states, self.inputs, self.ys = {}, {}, {}
        orig_capture, orig_inputs, orig_epi = hf.capture, hf.decode_inputs, hf.decode_epilogue

        def capture(m, cache_params, dt_min):
            self.states[m.layer_idx] = cache_params.layers[m.layer_idx].recurrent_states[0].detach().clone().cpu()
            self.inputs[m.layer_idx], self.ys[m.layer_idx] = [], []
            return orig_capture(m, cache_params, dt_min)

        def decode_inputs(m, *a):
            out = orig_inputs(m, *a)
            self.inputs[m.layer_idx].append([t.detach().clone().cpu() for t in out[1:]])
            return out

        def decode_epilogue(m, y, gate, dtype):
            self.ys[m.layer_idx].append(y.detach().clone().cpu())
            return orig_epi(m, y, gate, dtype)

        monkeypatch.setattr(hf, "capture", capture)
        monkeypatch.setattr(hf, "decode_inputs", decode_inputs)
        monkeypatch.setattr(hf, "decode_epilogue", decode_epilogue)


def _oracle_params(m, dt_min):
    from nested_ssm_amd import hf

    R = hf.mixer_rotation(m)
    return oracle.LayerParams(m.num_heads, m.head_dim, N, m.n_groups, m.dt_bias.detach().float().cpu(),
                              -torch.exp(m.A_log.detach().float()).cpu(), m.D.detach().float().cpu(),
                              None if R is None else R.float().cpu(), dt_min)


def _rot(S, R, H):
    Rh = R.double().repeat_interleave(H // R.shape[0], dim=0)
    return torch.einsum("bhpn,hmn->bhpm", S.double(), Rh).float()


def _replay_and_check(model, rec, pb, c, cold, dt_min_of, exact=False, modes=None):
    from nested_ssm_amd import hf

    for m in hf.mixers(model):
        li = m.layer_idx
        prm = _oracle_params(m, dt_min_of(m))
        S0 = rec.states[li]
        if prm.R is not None:
            S0 = _rot(S0, prm.R, m.num_heads)
        b = S0.shape[0]
        k = min(pb, N)
        ref = oracle.NativeV4(b, m.num_heads, m.head_dim, N, k, c, cold=cold, exact=exact)
        ref.join(torch.arange(b), S0)
        assert len(rec.inputs[li]) > 0
        for step, ((x, B, C, dt), y) in enumerate(zip(rec.inputs[li], rec.ys[li])):
            y_ref = ref.step(x, B, C, dt, prm, **(modes[step] if modes else {}))
            if cold == "fp32":
                assert_close32(y, y_ref, f"layer {li} step {step} (pb={pb}, c={c})")
            else:
                assert float((y - y_ref).norm() / y_ref.norm()) < 1e-4
        yield m, ref


def _prefill_decode(model, ids, n_decode):
    out = model(ids, use_cache=True)
    pkv = out.past_key_values
    logits = [out.logits[:, -1].float()]
    tok = out.logits[:, -1:].argmax(-1)
    for _ in range(n_decode):
        out = model(tok, past_key_values=pkv, use_cache=True)
        logits.append(out.logits[:, -1].float())
        tok = out.logits[:, -1:].argmax(-1)
    return torch.stack(logits, 1), pkv


@pytest.mark.parametrize("pb,c,cold_bf16", [(128, 16, 0), (32, 4, 0), (64, 3, 1), (16, 4, 0), (16, 16, 1)])
def test_native_install_matches_oracle(monkeypatch, pb, c, cold_bf16):
    from nested_ssm_amd import v4_native_decode as V

    V.M.is_fast_path_available = False  # the reference's callers set it; it must stay assignable
    model = _tiny_model(seed=3)
    assert V.install(model, pb=pb, c=c, cold_bf16=cold_bf16) == 2
    rec = Recorder(monkeypatch)
    ids = torch.randint(0, 96, (3, 9), generator=torch.Generator().manual_seed(4)).cuda()
    with torch.no_grad():
        _prefill_decode(model, ids, n_decode=2 * c + 1 if c < 16 else 6)
    cold = "bf16" if cold_bf16 and pb < N else "fp32"
    dt_min_of = lambda m: float(m.time_step_limit[0])  # noqa: E731
    for m, ref in _replay_and_check(model, rec, pb, c, cold, dt_min_of):
        st = m._v4state
        assert st["pb"] == pb and st["c"] == c
        if pb < N:
            assert st["t"] == int(ref.t[0])


@pytest.mark.parametrize("pb,c,cold_bf16", [(32, 4, 0), (64, 16, 1), (32, 32, 0)])
def test_native_install_corr_matches_oracle(monkeypatch, pb, c, cold_bf16):
    """install(..., corr=1): the rank-c exact correction readout
    (scale/v4_native_decode.py:81-117) against the oracle's exact mode (at c = 32 over the
    unit-blocked x ring the capture picks for it)."""
    from nested_ssm_amd import v4_native_decode as V

    model = _tiny_model(seed=11)
    assert V.install(model, pb=pb, c=c, cold_bf16=cold_bf16, corr=1) == 2
    rec = Recorder(monkeypatch)
    ids = torch.randint(0, 96, (3, 7), generator=torch.Generator().manual_seed(12)).cuda()
    with torch.no_grad():
        _prefill_decode(model, ids, n_decode=2 * c + 1)
    cold = "bf16" if cold_bf16 else "fp32"
    for m, ref in _replay_and_check(model, rec, pb, c, cold, lambda m: float(m.time_step_limit[0]), exact=True):
        assert m._v4state["t"] == int(ref.t[0])
        assert m._v4state["tier"].x_layout == (1 if c > 16 else 0)


def test_native_install_corr_gives_the_untiered_model():
    """With an fp32 cold tier, corr=1 reads the current cold state exactly, so the
    tiered model's logits equal the untiered (pb = N) install's up to fp32 rounding."""
    from nested_ssm_amd import v4_native_decode as V

    ids = torch.randint(0, 96, (2, 8), generator=torch.Generator().manual_seed(13)).cuda()
    with torch.no_grad():
        m_full = _tiny_model(seed=14)
        V.install(m_full, pb=128, c=4, cold_bf16=0)
        l_full, _ = _prefill_decode(m_full, ids, 9)
        m_corr = _tiny_model(seed=14)
        V.install(m_corr, pb=32, c=4, cold_bf16=0, corr=1)
        l_corr, _ = _prefill_decode(m_corr, ids, 9)
        m_stale = _tiny_model(seed=14)
        V.install(m_stale, pb=32, c=4, cold_bf16=0)
        l_stale, _ = _prefill_decode(m_stale, ids, 9)
    scale = l_full.abs().max()
    assert float((l_corr - l_full).abs().max() / scale) < 1e-4
    assert float((l_stale - l_full).abs().max() / scale) > 1e-4  # the stale readout is not exact


@pytest.mark.parametrize("master", ["bf16", "fp32"])
def test_fused_install_fp8_matches_oracle(monkeypatch, master):
    """install(cold="fp8") over the fused path's bf16 shadow master (the default) or an
    fp32 master: y within 2e-2 of the reference's fp8 emulation over the exact fp32
    state, and within 1e-4 of the oracle with the same master."""
    from nested_ssm_amd import v4_fused_decode as F

    model = _tiny_model(seed=5)
    kw = {} if master == "bf16" else dict(master=master)
    assert F.install(model, pb=32, c=4, cold="fp8", **kw) == 2
    for m in model.modules():
        if type(m).__name__ == "NemotronHMamba2Mixer":
            assert m._v4R is not None and m._v4R.dtype == torch.float32
    rec = Recorder(monkeypatch)
    ids = torch.randint(0, 96, (2, 6), generator=torch.Generator().manual_seed(6)).cuda()
    with torch.no_grad():
        _prefill_decode(model, ids, n_decode=9)
    from nested_ssm_amd import hf

    for m in hf.mixers(model):
        li = m.layer_idx
        prm = _oracle_params(m, 0.0)
        ref = oracle.NativeV4(2, m.num_heads, m.head_dim, N, 32, 4, cold="fp8")
        same = oracle.NativeV4(2, m.num_heads, m.head_dim, N, 32, 4, cold="fp8", master=master)
        S0 = _rot(rec.states[li], prm.R, m.num_heads)
        ref.join(torch.arange(2), S0)
        same.join(torch.arange(2), S0)
        for (x, B, C, dt), y in zip(rec.inputs[li], rec.ys[li]):
            y_ref = ref.step(x, B, C, dt, prm)
            y_same = same.step(x, B, C, dt, prm)
            assert float((y - y_ref).norm() / y_ref.norm()) <= 2e-2
            assert float((y - y_same).norm() / y_same.norm()) <= 1e-4


def test_all_hot_install_is_rotation_invariant_and_tracks_stock():
    """pb = N with a random orthogonal R gives the stock (unrotated) model's outputs:
    exactly up to fp32 rounding against the same install with R = I, and within
    the bf16 cast of the kernel inputs against the stock fp32 forward."""
    from nested_ssm_amd import v4_native_decode as V

    ids = torch.randint(0, 96, (2, 8), generator=torch.Generator().manual_seed(7)).cuda()
    with torch.no_grad():
        stock, _ = _prefill_decode(_tiny_model(seed=8, rotated=False), ids, 5)
        m_id = _tiny_model(seed=8, rotated=False)
        V.install(m_id, pb=128, c=16, cold_bf16=0)
        l_id, _ = _prefill_decode(m_id, ids, 5)
        m_rot = _tiny_model(seed=8, rotated=True)
        V.install(m_rot, pb=128, c=16, cold_bf16=0)
        l_rot, _ = _prefill_decode(m_rot, ids, 5)
    scale = stock.abs().max()
    assert float((l_rot - l_id).abs().max() / scale) < 1e-4
    assert float((l_id - stock).abs().max() / scale) < 2e-2
    assert torch.equal(l_id[:, 0], stock[:, 0])  # the prefill logits come from the stock forward


def test_restore_after_decode_gives_exact_state(monkeypatch):
    """A multi-token call after tiered decode tokens rebuilds the exact state
    (rotated back to the stock basis) in the cache before the stock forward."""
    from nested_ssm_amd import hf
    from nested_ssm_amd import v4_native_decode as V

    model = _tiny_model(seed=9)
    V.install(model, pb=32, c=4, cold_bf16=0)
    rec = Recorder(monkeypatch)
    restored = {}
    orig_restore = hf.restore_cache

    def restore(m, cache_params):
        orig_restore(m, cache_params)
        restored[m.layer_idx] = cache_params.layers[m.layer_idx].recurrent_states[0].detach().clone().cpu()

    monkeypatch.setattr(hf, "restore_cache", restore)
    ids = torch.randint(0, 96, (2, 5), generator=torch.Generator().manual_seed(10)).cuda()
    with torch.no_grad():
        _, pkv = _prefill_decode(model, ids, n_decode=6)
        rec_inputs = {k: list(v) for k, v in rec.inputs.items()}
        rec_states = dict(rec.states)
        model(ids[:, :2], past_key_values=pkv, use_cache=True)  # two tokens continue the sequence
    for m in hf.mixers(model):
        li = m.layer_idx
        prm = _oracle_params(m, float(m.time_step_limit[0]))
        ref = oracle.NativeV4(2, m.num_heads, m.head_dim, N, 32, 4)
        ref.join(torch.arange(2), _rot(rec_states[li], prm.R, m.num_heads))
        for x, B, C, dt in rec_inputs[li]:
            ref.step(x, B, C, dt, prm)
        Rh = prm.R.double().repeat_interleave(m.num_heads // m.n_groups, dim=0)
        want = torch.einsum("bhpm,hmn->bhpn", ref.S.double(), Rh).float()  # back to the stock basis
        assert_close32(restored[li], want, f"restored state layer {li}")


def test_generate_runs_with_tiered_decode():
    from nested_ssm_amd import v4_native_decode as V

    model = _tiny_model(seed=11)
    V.install(model, pb=32, c=4, cold_bf16=1)
    ids = torch.randint(0, 96, (2, 6), generator=torch.Generator().manual_seed(12)).cuda()
    with torch.no_grad():
        g1 = model.generate(ids, max_new_tokens=9, do_sample=False)
        g2 = model.generate(ids, max_new_tokens=9, do_sample=False)
    assert g1.shape == (2, 15) and torch.equal(g1, g2)


def _decode_with_modes(model, ids, modes):
    """Prefill, then one decode token per entry of modes, switching the mixers'
    v4cfg["coldoff"] / v4cfg["qgate"] before each (as scale/probe_selfspec_policy.py:125-136
    and scale/run_recall_native.py:85-89 mutate them)."""
    from nested_ssm_amd import hf

    out = model(ids, use_cache=True)
    pkv = out.past_key_values
    tok = out.logits[:, -1:].argmax(-1)
    for md in modes:
        for m in hf.mixers(model):
            m.v4cfg["coldoff"] = int(md.get("hot_only", False))
            m.v4cfg["qgate"] = md.get("qgate", 0.0)
        out = model(tok, past_key_values=pkv, use_cache=True)
        tok = out.logits[:, -1:].argmax(-1)
    return pkv


@pytest.mark.parametrize("cold_bf16", [0, 1])
def test_native_install_gated_readouts_match_oracle(monkeypatch, cold_bf16):
    """coldoff and qgate switched per token on the installed mixers against the oracle's
    gated readouts; the qgate counters read as scale/run_recall_native.py:116-118 does."""
    from nested_ssm_amd import hf
    from nested_ssm_amd import v4_native_decode as V

    pb, c = 32, 4
    model = _tiny_model(seed=21)
    assert V.install(model, pb=pb, c=c, cold_bf16=cold_bf16) == 2
    rec = Recorder(monkeypatch)
    ids = torch.randint(0, 96, (3, 7), generator=torch.Generator().manual_seed(22)).cuda()
    tau = (N - pb) / N
    modes = [[{}, dict(hot_only=True), dict(qgate=tau)][i % 3] for i in range(2 * c + 4)]
    with torch.no_grad():
        _decode_with_modes(model, ids, modes)
    cold = "bf16" if cold_bf16 else "fp32"
    for m, ref in _replay_and_check(model, rec, pb, c, cold, lambda m: float(m.time_step_limit[0]), modes=modes):
        st = m._v4state
        assert "qgate_n" in st and ref.qgate_n > 0
        assert st.get("qgate_n", 0) == ref.qgate_n and st.get("qgate_kept", 0) == ref.qgate_kept
        assert st["t"] == int(ref.t[0])
    with torch.no_grad():  # a new prompt's capture starts the counters again
        model(ids, use_cache=True)
    for m in hf.mixers(model):
        assert "qgate_n" not in m._v4state and m._v4state.get("qgate_kept", 0) == 0


def test_native_install_coldoff_with_an_unbounded_window(monkeypatch):
    """install(..., c=1 << 30, coldoff=1) (scale/probe_selfspec_alpha.py:59): the hot-only
    readout runs on the kernels' largest window, which it never reads, the state stays
    exact, and switching to the stale readout on that window is refused."""
    from nested_ssm_amd import v4_native_decode as V

    pb, c = 32, 1 << 30
    model = _tiny_model(seed=25)
    assert V.install(model, pb=pb, c=c, cold_bf16=0, coldoff=1) == 2
    rec = Recorder(monkeypatch)
    ids = torch.randint(0, 96, (2, 6), generator=torch.Generator().manual_seed(26)).cuda()
    modes = [dict(hot_only=True)] * 70  # past one 64-token window
    with torch.no_grad():
        pkv = _decode_with_modes(model, ids, modes)
    for m, ref in _replay_and_check(model, rec, pb, c, "fp32", lambda m: float(m.time_step_limit[0]),
                                    modes=modes):
        st = m._v4state
        assert dict.get(st, "tier").c == 64 and st["t"] == int(ref.t[0]) == len(modes)
        S = dict.get(st, "tier").materialize(st["params"]).cpu()
        assert_close32(S, ref.S, f"layer {m.layer_idx} state")
        assert st.get("qgate_n", 0) == 0 and "qgate_n" not in st
        m.v4cfg["coldoff"] = 0
    tok = torch.zeros(2, 1, dtype=torch.long, device="cuda")
    with torch.no_grad(), pytest.raises(NotImplementedError, match="coldoff"):
        model(tok, past_key_values=pkv, use_cache=True)


@pytest.mark.parametrize("corr,t_new", [(0, 1), (1, 3), (1, 0)])
def test_phase_write_mid_window_recaptures_the_tier(monkeypatch, corr, t_new):
    """Writing _v4state["t"] between decode tokens (scale/probe_selfspec_policy.py:127-128)
    mid-window: the tier is re-captured from its exact current state at the new phase, so
    the oracle replay re-joins there with its own current state; y at every token (stale or
    exact readout) and the final state match, and the phase reads back as written."""
    from nested_ssm_amd import hf
    from nested_ssm_amd import v4_native_decode as V

    pb, c = 32, 4
    model = _tiny_model(seed=31)
    assert V.install(model, pb=pb, c=c, cold_bf16=0, corr=corr) == 2
    rec = Recorder(monkeypatch)
    ids = torch.randint(0, 96, (3, 6), generator=torch.Generator().manual_seed(32)).cuda()
    n_before, n_after = 2, 2 * c + 3
    with torch.no_grad():
        out = model(ids, use_cache=True)
        pkv = out.past_key_values
        tok = out.logits[:, -1:].argmax(-1)
        for i in range(n_before + n_after):
            if i == n_before:
                for m in hf.mixers(model):
                    assert m._v4state["t"] == n_before  # mid-window: nv = 2 buffered tokens
                    m._v4state["t"] = t_new
                    assert m._v4state["t"] == t_new
            out = model(tok, past_key_values=pkv, use_cache=True)
            tok = out.logits[:, -1:].argmax(-1)
    for m in hf.mixers(model):
        li = m.layer_idx
        prm = _oracle_params(m, float(m.time_step_limit[0]))
        ref = oracle.NativeV4(3, m.num_heads, m.head_dim, N, pb, c, exact=bool(corr))
        ref.join(torch.arange(3), _rot(rec.states[li], prm.R, m.num_heads))
        for step, ((x, B, C, dt), y) in enumerate(zip(rec.inputs[li], rec.ys[li])):
            if step == n_before:
                ref.join(torch.arange(3), ref.S.clone(), phase=torch.full((3,), t_new))
            y_ref = ref.step(x, B, C, dt, prm)
            assert_close32(y, y_ref, f"layer {li} step {step} (corr={corr}, t <- {t_new})")
        tier = dict.get(m._v4state, "tier")
        assert_close32(tier.materialize(m._v4state["params"]).cpu(), ref.S, f"layer {li} state")
        assert m._v4state["t"] == t_new + n_after == int(ref.t[0])


@pytest.mark.parametrize("cfg,width", [(dict(mode="v4", c=4, pb=32), None), (dict(mode="v4", c=4, pb=32, cold_bf16=1), None),
                                       (dict(mode="v4", c=16, pb=16), None), (dict(mode="v4", c=3, pb=64, warm=5), None),
                                       (dict(mode="v4", c=4, pb=32, cold_fp8=1), None), (dict(mode="fresh"), None),
                                       (dict(mode="c1", c=4), None), (dict(mode="c1", c=16, cold_fp8=1), None),
                                       (dict(mode="c1", c=3, cold_bf16=1), None),
                                       (dict(mode="fresh"), 32), (dict(mode="v4", c=4, pb=32), 48),
                                       (dict(mode="c1", c=4), 64),
                                       (dict(mode="v4", c=4, pb=32, lag=1), None), (dict(mode="c1", c=3, lag=1), None),
                                       (dict(mode="v4", c=4, pb=32, cold_fp8=1, lag=1), None),
                                       (dict(mode="v4", c=16, pb=32, cold_bf16=1, lag=1), 48)])
def test_teacher_forced_state_op_matches_oracle(cfg, width):
    """The evaluation forward's state op (nemo9b_eval drop-in: one teacher-forced launch pair
    per token, sequences from zero states) against the oracle's restatement of
    scale/nemo9b_eval.py:41-85 on the same mixer inputs, modes "fresh", "v4" and "c1" (every
    column stale), with and without a width mask (set_width: the oracle masks the rotated
    B and C, the drop-in folds the mask into R), lag 0 and 1 (:44,59,70); fp32 1e-5, bf16
    snapshot the bf16 bar, e4m3 (per-row scale) 2e-2."""
    from helpers import assert_close_flips, max_rel
    from nested_ssm_amd import hf, nemo9b_eval as NE

    model = _tiny_model(seed=41)
    if width is not None:
        hf.set_width(model, width)
    m = hf.mixers(model)[0]
    full = dict(NE.CFG, **cfg)
    hidden = torch.randn(2, 13, 128, generator=torch.Generator().manual_seed(42)).cuda()
    with torch.no_grad():
        gate, x, B, C, dt = NE.teacher_forced_inputs(m, hidden)
        ys = NE.state_op(m, x, B, C, dt, full).cpu()
    prm = _oracle_params(m, float(m.time_step_limit[0]))
    k = N if full["mode"] == "fresh" else 0 if full["mode"] == "c1" else full["pb"]
    cold = "fp8" if full["cold_fp8"] else "bf16" if full["cold_bf16"] else "fp32"
    ref = oracle.TeacherForcedV4(2, m.num_heads, m.head_dim, N, k, full["c"], cold=cold, warm=full["warm"],
                                 lag=int(full["lag"]))
    ref.join(torch.arange(2), torch.zeros(2, m.num_heads, m.head_dim, N))
    for t in range(13):
        y_ref = ref.step(x[:, t].cpu(), B[:, t].cpu(), C[:, t].cpu(), dt[:, t].cpu(), prm, width=width)
        if cold == "fp8":
            assert max_rel(ys[:, t], y_ref) <= 2e-2
        elif cold == "bf16":
            assert_close_flips(ys[:, t], y_ref, f"token {t}")
        else:
            assert_close32(ys[:, t], y_ref, f"token {t} ({full})")


def test_teacher_forced_forward_tracks_the_stock_forward():
    """naive_mixer_forward bound to every mixer: mode "fresh" gives the stock forward's logits
    within the bf16 cast of the kernel inputs, v4 with pb = N is the fresh forward, and v4 with
    stale cold columns is not, nor its lagged form (lag = 1) the same; unsupported CFG keys
    raise."""
    from nested_ssm_amd import hf, nemo9b_eval as NE

    ids = torch.randint(0, 96, (2, 12), generator=torch.Generator().manual_seed(43)).cuda()
    model = _tiny_model(seed=44)
    with torch.no_grad():
        stock = model(ids, use_cache=False).logits.float()
        for m in hf.mixers(model):
            m.forward = NE.naive_mixer_forward.__get__(m)
        saved = dict(NE.CFG)
        try:
            NE.CFG.update(mode="fresh")
            fresh = model(ids, use_cache=False).logits.float()
            NE.CFG.update(mode="v4", c=4, pb=N)
            allhot = model(ids, use_cache=False).logits.float()
            NE.CFG.update(mode="v4", c=8, pb=32)
            v4 = model(ids, use_cache=False).logits.float()
            NE.CFG.update(mode="v4", lag=1)
            lagged = model(ids, use_cache=False).logits.float()
            NE.CFG.update(lag=0, state_bf16=1)
            with pytest.raises(NotImplementedError, match="state_bf16"):
                model(ids, use_cache=False)
        finally:
            NE.CFG.clear()
            NE.CFG.update(saved)
    scale = stock.abs().max()
    assert float((fresh - stock).abs().max() / scale) < 2e-2
    assert torch.equal(allhot, fresh)
    # stale cold columns move this small model's logits by ~1e-5 relative (fp32 rounding: ~1e-7)
    assert float((v4 - fresh).abs().max() / scale) > 5e-6
    assert not torch.equal(lagged, v4) and bool(torch.isfinite(lagged).all())


def test_reference_eval_driver_loop_runs_on_the_drop_in():
    """The evaluation driver of scale/nemo9b_eval.py:175-208 on the tiny model with
    naive_mixer_forward bound to every mixer: the validation forward, the ppl loop over modes
    ["c1", "v4"] and c, the needle arms fresh, hot-alone (set_width(model, pb)) and the mode
    loop again at full width. Every forward runs; c1 and v4 differ from fresh and from each
    other, hot-alone differs from fresh, and the full width restores the fresh logits (the
    numerics of each arm are checked against the oracle at the state op)."""
    from nested_ssm_amd import hf, nemo9b_eval as NE

    ids = torch.randint(0, 96, (2, 36), generator=torch.Generator().manual_seed(45)).cuda()  # c = 16 flushes twice
    model = _tiny_model(seed=46)
    pb, cs = 32, [4, 16]
    out = {}
    saved = dict(NE.CFG)
    try:
        with torch.no_grad():
            hf.set_width(model, 128)
            for m in hf.mixers(model):
                m.forward = NE.naive_mixer_forward.__get__(m)
            NE.CFG["mode"] = "fresh"
            out["fresh"] = model(ids, use_cache=False).logits.float()
            for mode in ["c1", "v4"]:
                for c in cs:
                    NE.CFG.update(mode=mode, c=c, pb=pb)
                    out[f"{mode}_c{c}"] = model(ids, use_cache=False).logits.float()
            NE.CFG.update(mode="fresh")
            out["needle_fresh"] = model(ids, use_cache=False).logits.float()
            hf.set_width(model, pb)  # hot-alone: the cold columns discarded
            out["needle_hotalone"] = model(ids, use_cache=False).logits.float()
            hf.set_width(model, 128)
            for mode in ["c1", "v4"]:
                for c in cs:
                    NE.CFG.update(mode=mode, c=c, pb=pb)
                    out[f"needle_{mode}_c{c}"] = model(ids, use_cache=False).logits.float()
    finally:
        NE.CFG.clear()
        NE.CFG.update(saved)
    for name, v in out.items():
        assert bool(torch.isfinite(v).all()), name
    scale = out["fresh"].abs().max()
    gap = lambda a, b: float((out[a] - out[b]).abs().max() / scale)  # noqa: E731
    assert torch.equal(out["needle_fresh"], out["fresh"])
    assert gap("needle_hotalone", "fresh") > 5e-6
    for c in cs:
        for arm in (f"c1_c{c}", f"v4_c{c}"):
            assert gap(arm, "fresh") > 5e-6 and gap(arm, "needle_hotalone") > 5e-6, arm
        assert gap(f"c1_c{c}", f"v4_c{c}") > 5e-6
        assert torch.equal(out[f"needle_c1_c{c}"], out[f"c1_c{c}"])
        assert torch.equal(out[f"needle_v4_c{c}"], out[f"v4_c{c}"])
