"""A decode step captured in a HIP graph (through torch.cuda.CUDAGraph): the attention layer as
the fused K+V pack and the decode attention, as the one call that packs and attends
(lq_int4_decode_attention_pack), both with split-K partials in the per-stream workspace, or as
the K+V pack and lq_int4_decode_attention_noalloc (partials in the library's static scratch; its
first call on the device, which resolves the scratch address, is the warm-up before the
capture), and an MX4 state update with the counter generator. Three replays, with eager GPU work and synchronizations between them, each
match the same calls run eagerly, bit for bit. None of these entry points records a memset."""
import pytest
import torch

from layer_quant_amd import _abi

pytestmark = pytest.mark.gpu


def _make_state(gpu, seed):
    gen = torch.Generator(device=gpu).manual_seed(seed)
    b, hkv, nrep, s, d, g = 2, 8, 4, 1000, 128, 32   # B * Hkv = 16: several key splits
    cap = s + 8
    t = dict(
        kp=torch.randint(0, 256, (b, hkv, cap, d // 2), dtype=torch.uint8, device=gpu, generator=gen),
        vp=torch.randint(0, 256, (b, hkv, cap, d // 2), dtype=torch.uint8, device=gpu, generator=gen),
        ks=torch.rand(b, hkv, cap, d // g, device=gpu, generator=gen) + 0.01,
        vs=torch.rand(b, hkv, cap, d // g, device=gpu, generator=gen) + 0.01,
        k_new=torch.randn(b, hkv, 1, d, device=gpu, generator=gen).to(torch.bfloat16),
        v_new=torch.randn(b, hkv, 1, d, device=gpu, generator=gen).to(torch.bfloat16),
        pos=torch.tensor([s - 1], device=gpu),
        q=torch.randn(b, hkv * nrep, 1, d, device=gpu, generator=gen).to(torch.bfloat16),
        att=torch.empty(b, hkv * nrep, d, device=gpu),
    )
    bsz, nh, p_, n, ng = 2, 16, 64, 128, 2
    h0 = torch.randn(bsz, nh, p_, n, device=gpu, generator=gen) * 0.5
    st = (torch.empty(bsz, nh, p_, n, dtype=torch.int8, device=gpu),
          torch.empty(bsz, nh, p_, n // 16, dtype=torch.uint8, device=gpu),
          torch.empty(bsz, nh, p_, n // 2, dtype=torch.uint8, device=gpu))
    _abi.mx_encode(h0, *st, 4, _abi.ROUND_NEAREST_EVEN)
    t.update(
        st=st,
        x=torch.randn(bsz, nh, p_, device=gpu, generator=gen).to(torch.bfloat16),
        dt=torch.randn(bsz, nh, device=gpu, generator=gen).to(torch.bfloat16)[:, :, None].expand(bsz, nh, p_),
        A=(-torch.exp(torch.rand(nh, device=gpu, generator=gen) * 2))[:, None, None].expand(nh, p_, n),
        B=torch.randn(bsz, ng, n, device=gpu, generator=gen).to(torch.bfloat16),
        C=torch.randn(bsz, ng, n, device=gpu, generator=gen).to(torch.bfloat16),
        D=torch.randn(nh, device=gpu, generator=gen)[:, None].expand(nh, p_),
        dt_bias=(torch.randn(nh, device=gpu, generator=gen) * 0.1)[:, None].expand(nh, p_),
        y=torch.empty(bsz, nh, p_, device=gpu, dtype=torch.bfloat16),
    )
    t["dims"] = (s, nrep, g)
    return t


def _step(t):
    s, nrep, g = t["dims"]
    if t["mode"] == "noalloc":
        _abi.int4_pack_kv_pair(t["k_new"], t["v_new"], t["kp"], t["vp"], t["ks"], t["vs"],
                               t["pos"], g)
        _abi.int4_decode_attention_noalloc(t["q"], t["kp"], t["vp"], t["ks"], t["vs"], None,
                                           t["att"], s, nrep, g)
    elif t["mode"] == "fused":
        _abi.int4_decode_attention_pack(t["q"], t["k_new"], t["v_new"], t["kp"], t["vp"], t["ks"],
                                        t["vs"], None, t["att"], s, nrep, g)
    else:
        _abi.int4_pack_kv_pair(t["k_new"], t["v_new"], t["kp"], t["vp"], t["ks"], t["vs"],
                               t["pos"], g)
        _abi.int4_decode_attention(t["q"], t["kp"], t["vp"], t["ks"], t["vs"], None, t["att"], s,
                                   nrep, g)
    _abi.mx_state_update(*t["st"], t["x"], t["dt"], t["dt_bias"], t["A"], t["B"], t["C"], t["D"],
                         None, t["y"], 4, True, _abi.ROUND_SR_COUNTER, seed=1234, rng_offset=4096)


def _snapshot(t):
    return [x.clone() for x in (t["kp"], t["vp"], t["ks"], t["vs"], t["att"], t["y"], *t["st"])]


def _restore(t, snap):
    for dst, src in zip((t["kp"], t["vp"], t["ks"], t["vs"], t["att"], t["y"], *t["st"]), snap):
        dst.copy_(src)


@pytest.mark.parametrize("mode", ["pack+attention", "fused", "noalloc"])
def test_decode_step_graph_replays_match_eager(gpu, mode):
    t = _make_state(gpu, 2024)
    t["mode"] = mode
    s, nrep, g = t["dims"]
    b, hkv, _, half_d = t["kp"].shape
    # several key splits, so that the partials (workspace or static scratch) are used
    assert _abi.lib().lq_int4_decode_attention_workspace(b, hkv * nrep, hkv, 2 * half_d, s, g) > 0
    start = _snapshot(t)
    eager = []
    for _ in range(3):  # the state update feeds the next step's state
        _step(t)
        torch.cuda.synchronize()
        eager.append(_snapshot(t))

    # warm up on a side stream (torch's recommended order), then capture from the start state
    _restore(t, start)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _step(t)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _step(t)
    torch.cuda.synchronize()

    _restore(t, start)
    torch.cuda.synchronize()
    junk = torch.randn(1 << 20, device=gpu)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        got = _snapshot(t)
        for a, b in zip(got, eager[i]):
            assert torch.equal(a, b), f"replay {i}"
        junk = junk * 1.0001 + 1.0  # eager work between replays
        torch.cuda.synchronize()
    assert torch.isfinite(t["att"]).all()


@pytest.mark.parametrize("rng", ["counter", "philox"])
@pytest.mark.parametrize("path", ["rows", "general"])
def test_device_step_graph_replays_draw_anew(gpu, diag, path, rng):
    """An MX4 stochastic update (the counter generator, or the reference's Philox stream)
    through the module with its step counter on the device (enable_device_step), captured
    together with the step's advance and replayed three times: the states are bit-identical to
    three eager host-offset updates at offsets 0, T and 2T (T = B*H*P*N), i.e. fresh draws on
    every replay, not three copies of one step's."""
    from hybrid_quant import mamba_state_8b_kernel as ms

    diag.set("LQ_MX_REQUIRE_ROWS" if path == "rows" else "LQ_MX_FORCE_GENERIC")
    mode = _abi.ROUND_SR_PHILOX if rng == "philox" else _abi.ROUND_SR_COUNTER
    t = _make_state(gpu, 99)
    bsz, nh, p_, n = t["st"][0].shape
    T = bsz * nh * p_ * n
    start = [a.clone() for a in t["st"]]

    def eager(offsets):
        st = [a.clone() for a in start]
        snaps = []
        for off in offsets:
            _abi.mx_state_update(*st, t["x"], t["dt"], t["dt_bias"], t["A"], t["B"], t["C"],
                                 t["D"], None, t["y"], 4, True, mode, seed=1234,
                                 rng_offset=off)
            torch.cuda.synchronize()
            snaps.append([a.clone() for a in st])
        return snaps

    want = eager([0, T, 2 * T])
    frozen = eager([0, 0, 0])
    assert not all(torch.equal(a, b) for a, b in zip(want[2], frozen[2]))  # offsets matter

    cache = ms.MambaStateKernelCache(*[a.clone() for a in start], format_bits=4)
    ms.enable_device_step(cache)

    def step():
        # dt_bias as the module reads it (with D's strides, ms.py:137): the same tensor here
        return ms.mx_state_selective_update(cache, t["x"], t["dt"], t["A"], t["B"], t["C"],
                                            D=t["D"], dt_bias=t["dt_bias"], dt_softplus=True,
                                            rng=rng)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm-up (advances the step; reset below)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    for dst, src in zip((cache.q_state, cache.shared_exp, cache.micro_exp), start):
        dst.copy_(src)
    cache.device_step.fill_(0)
    torch.cuda.synchronize()
    junk = torch.randn(1 << 20, device=gpu)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        got = (cache.q_state, cache.shared_exp, cache.micro_exp)
        for a, b in zip(got, want[i]):
            assert torch.equal(a, b), f"replay {i}"
        assert int(cache.device_step.item()) == i + 1
        junk = junk * 1.0001 + 1.0  # eager work between replays
        torch.cuda.synchronize()
