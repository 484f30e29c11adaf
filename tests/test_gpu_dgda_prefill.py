"""DGDA prefill on the GPU vs the oracle: the chunked MFMA path (per-token gates, dk = dv
= 64, bf16 q/k/v) and the sub-chunk MFMA path (per-channel gates, every head size in
{32, 64, 128}, bf16, fp16 and fp32).

Tolerance: rtol = atol = 2e-3 on fp32 outputs and final states for bf16 inputs
with fp32 accumulation.  bf16 outputs are checked to be
the rounding of the fp32 results.  The full BASELINE shape (B=4, H=10,
T=32768) is checked against the C oracle on two heads and through a
size-independent property on all of them: a prefill split in two halves and
chained through ``initial_state`` reproduces the single prefill.
"""
import numpy as np
import pytest
import torch

from _helpers import assert_close, dgda_inputs, oracle_dgda_args, to_np
from oracle import dgda as odgda
from oracle import dgda_c

pytestmark = pytest.mark.gpu


def _hip():
    from maba_sparse.kernels import hip_backend
    return hip_backend


def _run(inp, **kw):
    return _hip().hip_dgda_prefill(**inp, out_dtype=kw.pop("out_dtype", torch.float32),
                                   state_dtype=torch.float32, allow_mixed_dtypes=True, **kw)


def test_chunk_path_is_selected(dev):
    from maba_sparse import _native as N
    inp = dgda_inputs(1, 2, 4096, seed=0, device=dev)
    lib = N.load()
    n = lib.maba_hip_dgda_prefill_workspace_size(N.desc(inp["q"]), N.desc(inp["v"]), N.desc(inp["log_alpha"]),
                                                 N.desc(inp["b"]))
    assert n > 16          # multi-segment chunked path needs aggregate workspace
    inp["b"] = inp["b"].contiguous()   # per-channel erase gate -> sub-chunk path, also segmented
    n2 = lib.maba_hip_dgda_prefill_workspace_size(N.desc(inp["q"]), N.desc(inp["v"]), N.desc(inp["log_alpha"]),
                                                  N.desc(inp["b"]))
    assert n2 > 16
    small = dgda_inputs(1, 2, 4096, dk=32, dv=32, seed=0, device=dev)   # other head sizes -> sub-chunk path
    n3 = lib.maba_hip_dgda_prefill_workspace_size(N.desc(small["q"]), N.desc(small["v"]),
                                                  N.desc(small["log_alpha"]), N.desc(small["b"]))
    assert n3 > 16
    odd = dgda_inputs(1, 2, 4096, dk=48, dv=48, seed=0, device=dev)     # no MFMA path: sequential kernel
    n4 = lib.maba_hip_dgda_prefill_workspace_size(N.desc(odd["q"]), N.desc(odd["v"]),
                                                  N.desc(odd["log_alpha"]), N.desc(odd["b"]))
    assert n4 == 0


@pytest.mark.parametrize("decay", ["baseline", "slow", "none"])
@pytest.mark.parametrize("L", [1, 63, 64, 65, 200, 1024, 1025, 3000])
def test_chunk_vs_oracle(dev, decay, L):
    inp = dgda_inputs(1, 2, L, seed=L, decay=decay, device=dev, with_state=(L % 2 == 1))
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, f"out L={L} {decay}")
    assert_close(S, eS, 2e-3, 2e-3, f"state L={L} {decay}")


def test_chunk_alpha_instead_of_log_alpha(dev):
    inp = dgda_inputs(2, 2, 700, seed=4, device=dev)
    la = inp.pop("log_alpha")
    inp["alpha"] = torch.exp(la[..., :1]).expand(la.shape)   # per-token, stride-0 broadcast
    o, S = _run(inp)
    args = oracle_dgda_args({**inp, "log_alpha": la})
    eo, eS = odgda.dgda_prefill_seq(**args)
    assert_close(o, eo, 2e-3, 2e-3, "out")
    assert_close(S, eS, 2e-3, 2e-3, "state")


def test_chunk_per_channel_write_gate(dev):
    inp = dgda_inputs(1, 3, 300, seed=5, device=dev)
    inp["w"] = torch.rand(1, 3, 300, 64, generator=torch.Generator().manual_seed(1)).to(dev)
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, "out")
    assert_close(S, eS, 2e-3, 2e-3, "state")


def test_chunk_bf16_output_is_rounded_fp32(dev):
    inp = dgda_inputs(2, 2, 1500, seed=6, device=dev)
    o32, _ = _run(inp)
    o16, _ = _run(inp, out_dtype=torch.bfloat16)
    assert o16.dtype == torch.bfloat16
    assert torch.equal(o16, o32.to(torch.bfloat16))


def test_chunk_transposed_views(dev):
    """q/k/v as [B,L,H,d] storage viewed [B,H,L,d], as the DGDA layer passes them."""
    B, L, H = 2, 777, 3
    g = torch.Generator().manual_seed(8)
    mk = lambda: torch.nn.functional.normalize(torch.randn(B, L, H, 64, generator=g), dim=-1)
    q, k = (mk().bfloat16().to(dev).transpose(1, 2) for _ in range(2))
    v = torch.randn(B, L, H, 64, generator=g).bfloat16().to(dev).transpose(1, 2)
    la = (-torch.nn.functional.softplus(torch.randn(B, L, H, 1, generator=g) + 2)).to(dev).transpose(1, 2)
    be = torch.sigmoid(torch.randn(B, L, H, 1, generator=g)).to(dev).transpose(1, 2)
    inp = dict(q=q, k=k, v=v, log_alpha=la.expand(B, H, L, 64), b=be.expand(B, H, L, 64),
               w=be.expand(B, H, L, 64), initial_state=None)
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, "out")
    assert_close(S, eS, 2e-3, 2e-3, "state")


def test_baseline_shape_two_heads_vs_c_oracle(dev):
    """T = 32768 on (B=1, H=2) against the C chunked oracle (fp32)."""
    inp = dgda_inputs(1, 2, 32768, seed=2, device=dev)
    o, S = _run(inp)
    f = lambda t: to_np(t).astype(np.float32)
    eo, eS = dgda_c.dgda_prefill_chunked_c(f(inp["q"]), f(inp["k"]), f(inp["v"]), f(inp["log_alpha"][..., :1]),
                                           f(inp["b"][..., :1]), f(inp["w"][..., :1]), chunk_size=64)
    assert_close(o, eo, 2e-3, 2e-3, "out")
    assert_close(S, eS, 2e-3, 2e-3, "state")


@pytest.mark.parametrize("decay", ["baseline", "slow"])
def test_baseline_shape_split_chaining(dev, decay):
    """Full BASELINE config 2 shape: prefill(T) == prefill(T/2) -> prefill(T/2, initial_state).
    With the BASELINE decay the segment transitions vanish within a chunk or two (the
    zero-start pass and the gate-bound skip carry the run); with the slow decay none does
    (aggregate, zero-start and fix-up passes all do full work)."""
    B, H, T = 4, 10, 32768
    print(f"\nconfig 2 split chaining: decay={decay}", flush=True)
    inp = dgda_inputs(B, H, T, seed=3, decay=decay, device=dev)
    o, S = _run(inp)
    assert torch.isfinite(o).all() and torch.isfinite(S).all()
    h = T // 2
    first = {k: (v[:, :, :h] if (v is not None and v.dim() == 4 and k != "initial_state") else v) for k, v in inp.items()}
    second = {k: (v[:, :, h:] if (v is not None and v.dim() == 4 and k != "initial_state") else v) for k, v in inp.items()}
    o1, S1 = _run(first)
    second["initial_state"] = S1
    o2, S2 = _run(second)
    assert_close(torch.cat([o1, o2], dim=2), to_np(o), 2e-3, 2e-3, "chained out")
    assert_close(S2, to_np(S), 2e-3, 2e-3, "chained state")


def _slot_chunks(B, H, T):
    """Chunks per slot of the output pass at this shape on this device (U = max(16,
    ceil(chunks / (2 CUs)))), the slot cut of the zero-start launch."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    total = B * H * (T // 64)
    return max(16, -(-total // (2 * cus)))


def test_baseline_shape_full_run_heads_vs_c_oracle(dev):
    """The headline run itself -- B=4, H=10, T=32768, BASELINE decay, bf16 q/k/v, fp32
    per-token gates, bf16 output as the bench writes it -- with two of its heads against the
    C chunked oracle (fp32).  The heads are chosen so that their first chunk is not on a slot
    boundary: their segments start mid-slot, so every segment cut of those heads falls inside
    a sequence, their first segment runs in a slot shared with the previous head, and the
    gate-bound skip decides each later segment's start.  The bf16 output is the rounding of
    the same run's fp32 output."""
    B, H, T = 4, 10, 32768
    inp = dgda_inputs(B, H, T, seed=12, device=dev)
    U = _slot_chunks(B, H, T)
    nch = T // 64
    cut = [bh for bh in range(B * H) if (bh * nch) % U != 0]
    heads = [cut[0], cut[len(cut) // 2]]
    print(f"\nconfig 2 full run: U={U} heads (b*H+h)={heads}", flush=True)
    o16, S = _run(inp, out_dtype=torch.bfloat16)
    o32, S32 = _run(inp)
    assert torch.equal(o16, o32.to(torch.bfloat16))
    assert torch.equal(S, S32)
    f = lambda t: to_np(t).astype(np.float32)  # noqa: E731
    for bh in heads:
        b, h = divmod(bh, H)
        sl = lambda t: t[b:b + 1, h:h + 1]  # noqa: E731
        eo, eS = dgda_c.dgda_prefill_chunked_c(f(sl(inp["q"])), f(sl(inp["k"])), f(sl(inp["v"])),
                                               f(sl(inp["log_alpha"])[..., :1]), f(sl(inp["b"])[..., :1]),
                                               f(sl(inp["w"])[..., :1]), chunk_size=64)
        assert_close(sl(o32), eo, 2e-3, 2e-3, f"out head {bh}")
        assert_close(sl(S), eS, 2e-3, 2e-3, f"state head {bh}")


def test_chunk_mixed_decay_segments(dev):
    """Decay that is slow for the first 2600 tokens and fast afterwards, in one head, and
    the reverse in the other: segments whose transition vanishes after one or several
    chunks sit next to segments where it never does (zero-start, fix-up and full paths)."""
    L = 9000
    inp = dgda_inputs(1, 2, L, seed=77, device=dev, with_state=True)
    la = inp["log_alpha"][..., :1].clone()
    t = torch.arange(L, device=dev)
    slow = la * 0.005
    la[0, 0, :, 0] = torch.where(t < 2600, slow[0, 0, :, 0], la[0, 0, :, 0])
    la[0, 1, :, 0] = torch.where(t >= 6200, slow[0, 1, :, 0], la[0, 1, :, 0])
    inp["log_alpha"] = la.expand(1, 2, L, 64)
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, "out")
    assert_close(S, eS, 2e-3, 2e-3, "state")


@pytest.mark.parametrize("case", ["expanding_erase", "decay_above_one"])
def test_chunk_gate_bound_fallbacks(dev, case):
    """The aggregate pass skips a segment from its gates alone when the summed log-decay of its
    first chunks falls below -80 and every factor I - b k k^T is a contraction.  Erase gates
    of 2.6 on every 37th token (b |k|^2 > 2, a factor that expands) must send the segment to
    the exact test instead; decays above one on the first tokens of every chunk must count in
    the sum (here the sum still reaches the bound, a few tokens later)."""
    L = 4100
    inp = dgda_inputs(1, 2, L, seed=91, device=dev, with_state=True)
    t = torch.arange(L, device=dev)
    if case == "expanding_erase":
        b = inp["b"][..., :1].clone()
        b[:, :, t % 37 == 5] = 2.6
        inp["b"] = b.expand(1, 2, L, 64)
    else:
        la = inp["log_alpha"][..., :1].clone()
        la[:, :, t % 64 < 4] = 0.3
        inp["log_alpha"] = la.expand(1, 2, L, 64)
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, f"out {case}")
    assert_close(S, eS, 2e-3, 2e-3, f"state {case}")


@pytest.mark.parametrize("decay", ["baseline", "slow"])
def test_chunk_slot_boundaries_multi_head(dev, decay):
    """Six heads of 65 chunks: the output pass's 16-chunk slots start inside sequences
    and span two sequences, so segments of every length meet at the cuts."""
    inp = dgda_inputs(2, 3, 4100, seed=21, decay=decay, device=dev, with_state=True)
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, f"out {decay}")
    assert_close(S, eS, 2e-3, 2e-3, f"state {decay}")


def test_chunk_wide_slots_vs_c_oracle(dev):
    """36 heads of 256 chunks exceed 16 chunks per slot on 256 CUs (U = 18), so the cuts
    fall at sequence offsets that move from head to head; four heads are checked
    against the C chunked oracle."""
    inp = dgda_inputs(1, 36, 16384, seed=5, device=dev)
    o, S = _run(inp)
    heads = [0, 1, 17, 35]
    f = lambda t: to_np(t[:, heads]).astype(np.float32)  # noqa: E731
    eo, eS = dgda_c.dgda_prefill_chunked_c(f(inp["q"]), f(inp["k"]), f(inp["v"]), f(inp["log_alpha"][..., :1]),
                                           f(inp["b"][..., :1]), f(inp["w"][..., :1]), chunk_size=64)
    assert_close(o[:, heads], eo, 2e-3, 2e-3, "out")
    assert_close(S[:, heads], eS, 2e-3, 2e-3, "state")


# ----------------------------------------------------------------------------- per-channel gates
# Per-channel gates (the DGDA layer's layout) take the sub-chunk path: 16-token
# sub-chunks with exact per-channel decay (pair-by-pair exponentials when a sub-chunk's
# decay range is too wide for the MFMA factorisation), segments chained through
# aggregate and fix-up passes.

@pytest.mark.parametrize("qkv", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("decay", ["baseline", "slow", "none"])
@pytest.mark.parametrize("L", [1, 31, 33, 1000, 4100])
def test_subchunk_path_per_channel_gates(dev, qkv, decay, L):
    inp = dgda_inputs(2, 3, L, seed=L + 7, decay=decay, gates="channel", qkv_dtype=qkv, device=dev,
                      with_state=(L % 2 == 1))
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, f"out L={L} {decay} {qkv}")
    assert_close(S, eS, 2e-3, 2e-3, f"state L={L} {decay} {qkv}")


def test_subchunk_path_alpha_strong_decay_and_bf16_output(dev):
    """alpha instead of log_alpha, per-channel decays down to e^-30 per token (sub-chunks
    whose decay range exceeds the MFMA factorisation take the exact pair-by-pair form),
    bf16 output: bf16 outputs round the fp32 results."""
    L = 3000
    inp = dgda_inputs(1, 4, L, seed=31, gates="channel", device=dev, with_state=True)
    la = inp.pop("log_alpha")
    la = torch.where(torch.rand(la.shape, generator=torch.Generator().manual_seed(1)).to(dev) < 0.1, la * 15, la)
    inp["alpha"] = torch.exp(la)
    o32, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args({**inp, "log_alpha": la}))
    assert_close(o32, eo, 2e-3, 2e-3, "out")
    assert_close(S, eS, 2e-3, 2e-3, "state")
    o16, _ = _run(inp, out_dtype=torch.bfloat16)
    assert torch.equal(o16, o32.to(torch.bfloat16))


def test_subchunk_path_growing_gates_never_vanish(dev):
    """log_alpha > 0 on some channels: the segment transitions never vanish, so every
    segment after the first runs in the fix-up pass from a scanned start state."""
    L = 6000
    inp = dgda_inputs(1, 2, L, seed=41, decay="slow", gates="channel", device=dev)
    la = inp["log_alpha"].clone()
    la[..., :4] = 0.0005            # four channels that grow slowly
    inp["log_alpha"] = la
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, "out")
    assert_close(S, eS, 2e-3, 2e-3, "state")


def test_subchunk_path_config2_shape_split_chaining(dev):
    """Config-2 shape with per-channel gates (B=4, H=10, T=32768): prefill(T) equals
    prefill(T/2) chained into prefill(T/2, initial_state), and two heads match the
    token-loop oracle over the first 4096 tokens."""
    B, H, T = 4, 10, 32768
    inp = dgda_inputs(B, H, T, seed=9, gates="channel", device=dev)
    o, S = _run(inp)
    assert torch.isfinite(o).all() and torch.isfinite(S).all()
    h = T // 2
    part = lambda sl: {k: (v[:, :, sl] if (v is not None and v.dim() == 4 and k != "initial_state") else v)  # noqa: E731
                       for k, v in inp.items()}
    o1, S1 = _run(part(slice(0, h)))
    second = part(slice(h, T))
    second["initial_state"] = S1
    o2, S2 = _run(second)
    assert_close(torch.cat([o1, o2], dim=2), to_np(o), 2e-3, 2e-3, "chained out")
    assert_close(S2, to_np(S), 2e-3, 2e-3, "chained state")
    few = {k: (v[:1, :2, :4096] if (v is not None and v.dim() == 4 and k != "initial_state") else v)
           for k, v in inp.items()}
    eo, _ = odgda.dgda_prefill_seq(**oracle_dgda_args(few))
    assert_close(o[:1, :2, :4096], eo, 2e-3, 2e-3, "oracle heads")


# ----------------------------------------------------------------------------- head sizes and dtypes
# Every head size the reference's GPU prefill takes (d_k, d_v in {32, 64, 128},
# triton_dgda.py:389-396) runs on the sub-chunk MFMA path; d_v = 128 as two calls over the
# halves of the value columns.  Each case asserts that path from its workspace size (the
# sequential kernel takes none) and spans at least two segments, so the aggregate and
# fix-up passes run: "baseline" decay lets every segment map vanish, "slow" keeps them
# alive, "strong" adds decays down to e^-30 per token (pair-by-pair sub-chunks).

def _sub_workspace_size(inp):
    from maba_sparse import _native as N
    lib = N.load()
    return lib.maba_hip_dgda_prefill_workspace_size(N.desc(inp["q"]), N.desc(inp["v"]), N.desc(inp["log_alpha"]),
                                                    N.desc(inp["b"]))


def _expected_sub_workspace(B, H, L, dk, dv, cus):
    """Slots of U = max(64, ceil(B*H*nch / (2 CUs))) sub-chunks of 16 tokens; a sequence of nch
    > U sub-chunks spans at most ceil((nch - 1) / U) + 1 segments, each holding a d_k x
    (d_v + d_k) fp32 segment map (d_v of one call: 64 when d_v = 128) and an int32 count."""
    nch = -(-L // 16)
    U = max(64, -(-B * H * nch // (2 * cus)))
    nseg = 1 if nch <= U else -(-(nch - 1) // U) + 1
    dvc = 64 if dv == 128 else dv
    return B * H * nseg * (dk * (dvc + dk) * 4 + 4), nseg


@pytest.mark.parametrize("dk,dv", [(32, 32), (32, 64), (32, 128), (64, 32), (64, 128), (128, 32), (128, 64),
                                   (128, 128)])
@pytest.mark.parametrize("decay,L,qkv", [("baseline", 1100, torch.bfloat16), ("slow", 3000, torch.float32),
                                         ("strong", 2100, torch.bfloat16)])
def test_subchunk_head_sizes_vs_oracle(dev, dk, dv, decay, L, qkv):
    B, H = 1, 2
    inp = dgda_inputs(B, H, L, dk=dk, dv=dv, seed=dk + 3 * dv + L, decay="baseline" if decay == "strong" else decay,
                      gates="channel", qkv_dtype=qkv, device=dev, with_state=(decay != "baseline"))
    if decay == "strong":
        la = inp["log_alpha"]
        pick = torch.rand(la.shape, generator=torch.Generator().manual_seed(5)).to(dev) < 0.1
        inp["log_alpha"] = torch.where(pick, la * 15, la)
    n = _sub_workspace_size(inp)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    want, nseg = _expected_sub_workspace(B, H, L, dk, dv, cus)
    assert nseg >= 2 and n == want and n > 16, (n, want, nseg)
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, f"out dk={dk} dv={dv} {decay}")
    assert_close(S, eS, 2e-3, 2e-3, f"state dk={dk} dv={dv} {decay}")


@pytest.mark.parametrize("dk,dv,L,qkv", [(128, 32, 1, torch.float16), (32, 128, 15, torch.bfloat16),
                                         (128, 128, 17, torch.float32), (32, 32, 16, torch.float16)])
def test_subchunk_head_sizes_short_sequences(dev, dk, dv, L, qkv):
    """One sub-chunk or a partial one (L = 1, 15, 16, 17) at the other head sizes, with an initial
    state: a single segment, the zero-start pass alone, masked tail tokens."""
    inp = dgda_inputs(2, 3, L, dk=dk, dv=dv, seed=L + dk, gates="channel", qkv_dtype=qkv, device=dev,
                      with_state=True)
    assert _sub_workspace_size(inp) == 16            # one slot per sequence: no aggregate workspace
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, f"out dk={dk} dv={dv} L={L}")
    assert_close(S, eS, 2e-3, 2e-3, f"state dk={dk} dv={dv} L={L}")


@pytest.mark.parametrize("dk,dv", [(128, 128), (32, 64)])
def test_subchunk_head_sizes_views_and_token_gates(dev, dk, dv):
    """q/k/v as [B,L,H,d] storage viewed [B,H,L,d] (the layer's layout), per-token gates as stride-0
    channel views (shared by both value halves at d_v = 128), many segments per sequence."""
    B, L, H = 2, 5000, 3
    g = torch.Generator().manual_seed(dk + dv)
    nrm = lambda t: torch.nn.functional.normalize(t, dim=-1)  # noqa: E731
    q = nrm(torch.randn(B, L, H, dk, generator=g)).bfloat16().to(dev).transpose(1, 2)
    k = nrm(torch.randn(B, L, H, dk, generator=g)).bfloat16().to(dev).transpose(1, 2)
    v = torch.randn(B, L, H, dv, generator=g).bfloat16().to(dev).transpose(1, 2)
    la = (-torch.nn.functional.softplus(torch.randn(B, H, L, 1, generator=g) + 2) * 0.01).to(dev)
    be = torch.sigmoid(torch.randn(B, H, L, 1, generator=g)).to(dev)
    inp = dict(q=q, k=k, v=v, log_alpha=la.expand(B, H, L, dk), b=be.expand(B, H, L, dk),
               w=be.expand(B, H, L, dv), initial_state=None)
    if dk != 64 or dv != 64:
        assert _sub_workspace_size(inp) > 16
    o, S = _run(inp)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, "out")
    assert_close(S, eS, 2e-3, 2e-3, "state")


@pytest.mark.parametrize("dk,dv", [(64, 64), (32, 128), (128, 32)])
def test_subchunk_fp16_same_dtype_contract(dev, dk, dv):
    """Every tensor fp16 (the reference's contract without mixed dtypes: gates in q's dtype),
    through the dispatcher with chunk_size 16: fp16 output and state within 2e-3 of the
    float64 recurrence on the fp16-rounded inputs, and the fp16 output is the rounding of
    the kernel's fp32 result (fp32 output requested from the same fp16 inputs)."""
    from maba_sparse.kernels.dispatcher import dispatch_dgda_prefill
    B, H, L = 1, 3, 1500
    inp = dgda_inputs(B, H, L, dk=dk, dv=dv, seed=dk * dv, decay="slow", gates="channel", qkv_dtype=torch.float16,
                      gate_dtype=torch.float16, device=dev, with_state=True)
    inp["initial_state"] = inp["initial_state"].half()
    assert _sub_workspace_size(inp) > 16
    o, S = dispatch_dgda_prefill(**inp, chunk_size=16)
    assert o.dtype == torch.float16 and S.dtype == torch.float16
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 2e-3, 2e-3, "fp16 out")
    assert_close(S, eS, 2e-3, 2e-3, "fp16 state")
    o32, _ = _hip().hip_dgda_prefill(**inp, out_dtype=torch.float32, state_dtype=torch.float32)
    assert torch.equal(o, o32.to(torch.float16))


def test_subchunk_bf16_gates(dev):
    """bf16 q, k, v and bf16 gates (16-bit gate loads), per-token and per-channel."""
    for gates in ("scalar", "channel"):
        inp = dgda_inputs(2, 2, 1200, seed=77, decay="slow", gates=gates, gate_dtype=torch.bfloat16, device=dev)
        assert _sub_workspace_size(inp) > 16
        o, S = _run(inp)
        eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
        assert_close(o, eo, 2e-3, 2e-3, f"out {gates}")
        assert_close(S, eS, 2e-3, 2e-3, f"state {gates}")


# ----------------------------------------------------------------------------- config 1
def _config1_inputs(device):
    """B=1, H=10, T=2048, d=64, fp32; per-token gates as the op's
    ``[B,H,T,64]`` stride-0 views, both decay forms given (the reference layer's call)."""
    inp = dgda_inputs(1, 10, 2048, qkv_dtype=torch.float32, seed=101, device=device)
    inp["alpha"] = torch.exp(inp["log_alpha"][..., :1]).expand(inp["log_alpha"].shape)
    return inp


def test_config1_fp32_dispatch_vs_oracle(dev):
    """Config 1 at its shape through the dispatcher, every tensor fp32 (the reference's
    dtype contract, no mixed dtypes), chunk_size 16 as the layer passes it: rtol = atol =
    1e-4 against the float64 token recurrence (fp32 inputs, products carried to about 16
    mantissa bits by the hi/lo MFMA splits)."""
    from maba_sparse.kernels.dispatcher import dispatch_dgda_prefill
    inp = _config1_inputs(dev)
    o, S = dispatch_dgda_prefill(**inp, chunk_size=16)
    assert o.dtype == torch.float32 and S.dtype == torch.float32 and o.shape == (1, 10, 2048, 64)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    err = max(float(np.abs(to_np(o) - eo).max()), float(np.abs(to_np(S) - eS).max()))
    print(f"\nconfig 1 fp32: max abs error {err:.3e}", flush=True)
    assert_close(o, eo, 1e-4, 1e-4, "config 1 out")
    assert_close(S, eS, 1e-4, 1e-4, "config 1 state")


@pytest.mark.parametrize("gates", ["scalar", "channel"])
def test_growing_decay_contract_hip_vs_reference_backend(dev, gates):
    """Decays above one (log_alpha = +0.05 on every seventh token), log_alpha alone: the hip
    backend computes the token recurrence with the gates as given -- the reference's own
    ``reference`` backend (``ref_dgda_prefill``, common.py:229-268), run here by torch on the
    same GPU tensors in fp32 -- through the chunked path (per-token gates) and the sub-chunk
    path (per-channel gates).  The reference's CPU algorithm clamps in-chunk decay ratios to
    one and so differs for such gates (the ``cpu`` backend mirrors it; pinned in
    test_cpu_dgda.py)."""
    from maba_sparse.kernels.dispatcher import get_kernel
    inp = dgda_inputs(2, 3, 700, seed=17, gates=gates, device=dev, with_state=True)
    la = inp["log_alpha"][..., :1].clone() if gates == "scalar" else inp["log_alpha"].clone()
    la[:, :, ::7] = 0.05
    inp["log_alpha"] = la.expand(inp["log_alpha"].shape) if gates == "scalar" else la
    o, S = _run(inp)
    ref = get_kernel("reference", "dgda_prefill")
    f32 = {k: (v.float() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    ro, rS = ref(**f32)
    eo, eS = odgda.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(ro, eo, 1e-4, 1e-4, "reference backend vs the float64 recurrence")
    assert_close(o, to_np(ro), 2e-3, 2e-3, f"hip vs reference backend, {gates} gates")
    assert_close(S, to_np(rS), 2e-3, 2e-3, f"hip vs reference backend state, {gates} gates")
