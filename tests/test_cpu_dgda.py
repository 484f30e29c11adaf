"""The ``cpu`` backend's chunked DGDA (kernels/cpu_dgda.py) against the float64 token
recurrence of the oracle (``oracle.dgda.dgda_prefill_seq`` / ``dgda_step``).

Tolerance: fp32 inputs rtol = atol = 1e-4 (fp32 arithmetic against float64, chunk
products of 16-64 terms); bf16 inputs rtol = atol = 2e-2 on the bf16 results (one
rounding of the output to bf16 on top).  The "approximate" inversion is the reference's
third-order Neumann series, exact only while (L)^4 vanishes; it is checked on inputs with
a small erase gate, where the series' remainder is below the tolerance.
"""
import numpy as np
import pytest
import torch

from _helpers import assert_close, dgda_inputs, oracle_dgda_args, to_np
from oracle import dgda as od


def _cpu():
    from maba_sparse.kernels import cpu_dgda
    return cpu_dgda


@pytest.mark.parametrize("B,H,L,dk,dv,gates,decay,chunk,state", [
    (2, 3, 37, 16, 24, "channel", "baseline", 16, True),   # ragged tail, dk != dv
    (1, 2, 64, 32, 32, "scalar", "slow", 16, False),      # stride-0 gates, long memory
    (1, 1, 1, 8, 8, "channel", "none", 16, True),         # one token
    (2, 2, 130, 64, 64, "channel", "slow", 64, True),     # chunk 64, several blocks' worth of chunks
])
@pytest.mark.parametrize("method", ["exact", "adaptive"])
def test_cpu_prefill_vs_oracle(B, H, L, dk, dv, gates, decay, chunk, state, method):
    inp = dgda_inputs(B, H, L, dk=dk, dv=dv, qkv_dtype=torch.float32, gates=gates, decay=decay, seed=L + dk,
                      with_state=state)
    o, S = _cpu().cpu_dgda_prefill(**inp, chunk_size=chunk, inversion_method=method)
    eo, eS = od.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert o.dtype == torch.float32 and S.dtype == torch.float32
    assert_close(o, eo, 1e-4, 1e-4, f"out {method}")
    assert_close(S, eS, 1e-4, 1e-4, f"state {method}")


def test_cpu_prefill_approximate_inverse_small_erase():
    inp = dgda_inputs(1, 2, 100, dk=16, dv=16, qkv_dtype=torch.float32, gates="channel", seed=3)
    inp["b"] = inp["b"] * 0.05          # |L| small: the Neumann series' remainder is negligible
    o, S = _cpu().cpu_dgda_prefill(**inp, inversion_method="approximate")
    eo, eS = od.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 1e-4, 1e-4, "out")
    assert_close(S, eS, 1e-4, 1e-4, "state")


def test_cpu_prefill_bf16_alpha_and_block_split(monkeypatch):
    """bf16 inputs come back in bf16; alpha instead of log_alpha gives the same result; a
    block bound of one chunk (every block one chunk long) changes nothing."""
    cd = _cpu()
    inp = dgda_inputs(1, 2, 200, dk=32, dv=32, qkv_dtype=torch.float32, gates="channel", seed=9, with_state=True)
    o, S = cd.cpu_dgda_prefill(**inp)
    la = inp.pop("log_alpha")
    o2, S2 = cd.cpu_dgda_prefill(**inp, alpha=torch.exp(la))
    assert torch.allclose(o, o2, rtol=1e-5, atol=1e-6) and torch.allclose(S, S2, rtol=1e-5, atol=1e-6)
    monkeypatch.setattr(cd, "_BLOCK_BYTES", 1)
    o3, S3 = cd.cpu_dgda_prefill(**inp, alpha=torch.exp(la))
    assert torch.allclose(o, o3, rtol=1e-5, atol=1e-6) and torch.allclose(S, S3, rtol=1e-5, atol=1e-6)
    bf = {k: (v.bfloat16() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    ob, Sb = cd.cpu_dgda_prefill(**bf, alpha=torch.exp(la).bfloat16())
    assert ob.dtype == torch.bfloat16 and Sb.dtype == torch.bfloat16
    eo, eS = od.dgda_prefill_seq(q=to_np(bf["q"]), k=to_np(bf["k"]), v=to_np(bf["v"]),
                                 alpha=to_np(torch.exp(la).bfloat16()), b=to_np(bf["b"]), w=to_np(bf["w"]),
                                 initial_state=to_np(bf["initial_state"]))
    assert_close(ob, eo, 2e-2, 2e-2, "bf16 out")
    assert_close(Sb, eS, 2e-2, 2e-2, "bf16 state")


def test_cpu_prefill_empty_and_step():
    cd = _cpu()
    inp = dgda_inputs(2, 2, 0, dk=8, dv=8, qkv_dtype=torch.float32, gates="channel", with_state=True)
    o, S = cd.cpu_dgda_prefill(**inp)
    assert o.shape == (2, 2, 0, 8) and torch.equal(S, inp["initial_state"])
    one = dgda_inputs(2, 3, 1, dk=8, dv=12, qkv_dtype=torch.float32, gates="channel", seed=4, with_state=True)
    s0 = one.pop("initial_state")
    o, S = cd.cpu_dgda_step(**one, state=s0)
    args = oracle_dgda_args(dict(one, initial_state=s0))
    eo, eS = od.dgda_step(args["q"][:, :, 0], args["k"][:, :, 0], args["v"][:, :, 0], alpha=args["alpha"][:, :, 0],
                          b=args["b"][:, :, 0], w=args["w"][:, :, 0], state=args["initial_state"])
    assert_close(o, eo, 1e-5, 1e-6, "step out")
    assert_close(S, eS, 1e-5, 1e-6, "step state")


def test_cpu_backend_selected_for_host_tensors():
    from maba_sparse.kernels import dispatcher as D
    from maba_sparse.kernels import cpu_dgda
    assert D.get_kernel("cpu", "dgda_prefill") is cpu_dgda.cpu_dgda_prefill
    assert D.get_kernel("cpu", "dgda_step") is cpu_dgda.cpu_dgda_step
    inp = dgda_inputs(1, 2, 50, dk=16, dv=16, qkv_dtype=torch.float32, gates="channel", seed=1)
    o, S = D.dispatch_dgda_prefill(**inp, chunk_size=16)
    eo, eS = od.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 1e-4, 1e-4, "dispatched out")
    assert np.isfinite(to_np(S)).all()


def test_cpu_backend_config1_shape():
    """BASELINE config 1 (B=1, H=10, T=2048, d=64, fp32, per-token gates, zero state) through
    the dispatcher on host tensors -- the ``cpu`` backend, chunk_size 16 and the adaptive
    inversion as the layer calls it -- against the float64 token recurrence."""
    from maba_sparse.kernels import dispatcher as D
    inp = dgda_inputs(1, 10, 2048, qkv_dtype=torch.float32, seed=101)
    inp["alpha"] = torch.exp(inp["log_alpha"][..., :1]).expand(inp["log_alpha"].shape)
    o, S = D.dispatch_dgda_prefill(**inp, chunk_size=16, inversion_method="adaptive", adaptive_tol=7e-5)
    assert o.shape == (1, 10, 2048, 64) and o.dtype == torch.float32
    eo, eS = od.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 1e-4, 1e-4, "config 1 out")
    assert_close(S, eS, 1e-4, 1e-4, "config 1 state")


def test_cpu_growing_decay_follows_reference_cpu_branches():
    """Decays above one (log_alpha > 0 on some tokens) take the reference CPU's branches
    (cpu_dgda.py:63-68, 101-103):
    - log_alpha alone is used as given.  With chunk_size 1 no decay ratio lies inside a chunk,
      so the chunked algorithm is the token recurrence itself: it must equal the float64
      recurrence on the unclamped gates;
    - alpha and log_alpha both given: log_alpha is clamped to [-46, 0], so the result is the
      recurrence on the clamped gates (no ratio then exceeds one, and the chunk size does
      not matter)."""
    inp = dgda_inputs(1, 2, 90, dk=16, dv=16, qkv_dtype=torch.float32, gates="channel", seed=5, with_state=True)
    la = inp["log_alpha"].clone()
    la[:, :, ::7] = 0.05                              # growing on every seventh token
    inp["log_alpha"] = la
    o, S = _cpu().cpu_dgda_prefill(**inp, chunk_size=1)
    eo, eS = od.dgda_prefill_seq(**oracle_dgda_args(inp))
    assert_close(o, eo, 1e-4, 1e-4, "log_alpha alone, chunk 1")
    assert_close(S, eS, 1e-4, 1e-4, "log_alpha alone, chunk 1 state")
    o2, S2 = _cpu().cpu_dgda_prefill(**inp, alpha=torch.exp(la), chunk_size=16)
    eo2, eS2 = od.dgda_prefill_seq(**oracle_dgda_args(dict(inp, log_alpha=la.clamp(-46.0, 0.0))))
    assert_close(o2, eo2, 1e-4, 1e-4, "both forms: clamped")
    assert_close(S2, eS2, 1e-4, 1e-4, "both forms: clamped state")
