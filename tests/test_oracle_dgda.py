"""Pins the DGDA oracle (CPU only).

Each check is chosen so that a plausible transcription mistake in the oracle
(a dropped decay, transposed state, wrong gate) fails it: hand-computed
golden vectors, the delta rule's exact-write property, the invariants the
reference tests assert (test_cpu_dgda.py:143-157, 210-230, 472-495;
test_triton_dgda.py:162-180; test_dgda.py:122-137) and a brute-force
matrix restatement on tiny shapes.
"""
import json
import os

import numpy as np
import pytest

from oracle import dgda as od
from oracle import dgda_c

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "dgda_golden.json")


def _rand(B, H, L, dk, dv, seed, decay=True):
    r = np.random.default_rng(seed)
    q = r.standard_normal((B, H, L, dk))
    k = r.standard_normal((B, H, L, dk))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = r.standard_normal((B, H, L, dv))
    a = np.exp(-np.log1p(np.exp(r.standard_normal((B, H, L, dk)) + 2))) if decay else np.ones((B, H, L, dk))
    b = 1 / (1 + np.exp(-r.standard_normal((B, H, L, dk))))
    w = 1 / (1 + np.exp(-r.standard_normal((B, H, L, dv))))
    return q, k, v, a, b, w


def test_golden_vectors():
    """Hand-computed cases stored under tests/golden (see make_golden.py for the arithmetic)."""
    with open(GOLDEN) as fh:
        cases = json.load(fh)
    assert cases
    for c in cases:
        arr = {k: np.array(v, np.float64) for k, v in c["inputs"].items()}
        o, S = od.dgda_prefill_seq(arr["q"], arr["k"], arr["v"], alpha=arr["alpha"], b=arr["b"], w=arr["w"],
                                   initial_state=arr.get("initial_state"))
        np.testing.assert_allclose(o, np.array(c["out"]), rtol=0, atol=1e-12, err_msg=c["name"])
        np.testing.assert_allclose(S, np.array(c["state"]), rtol=0, atol=1e-12, err_msg=c["name"])


def test_exact_write_of_delta_rule():
    """alpha = b = w = 1 and orthonormal keys: after writing (k_i, v_i) the state returns v_i exactly."""
    r = np.random.default_rng(0)
    dk, dv, L = 8, 5, 6
    Q, _ = np.linalg.qr(r.standard_normal((dk, dk)))
    k = Q[:L][None, None]
    v = r.standard_normal((1, 1, L, dv))
    ones_k, ones_v = np.ones((1, 1, L, dk)), np.ones((1, 1, L, dv))
    _, S = od.dgda_prefill_seq(k, k, v, alpha=ones_k, b=ones_k, w=ones_v)
    np.testing.assert_allclose(k[0, 0] @ S[0, 0], v[0, 0], atol=1e-12)
    # overwriting a key replaces its value
    v2 = r.standard_normal((1, 1, 1, dv))
    _, S2 = od.dgda_prefill_seq(k[:, :, :1], k[:, :, :1], v2, alpha=ones_k[:, :, :1], b=ones_k[:, :, :1],
                                w=ones_v[:, :, :1], initial_state=S)
    np.testing.assert_allclose(k[0, 0, 0] @ S2[0, 0], v2[0, 0, 0], atol=1e-12)
    np.testing.assert_allclose(k[0, 0, 1:] @ S2[0, 0], v[0, 0, 1:], atol=1e-12)


def test_zero_decay_wipes_initial_state():
    q, k, v, a, b, w = _rand(2, 2, 5, 4, 3, 1)
    a[:] = 0.0
    r = np.random.default_rng(9)
    o1, S1 = od.dgda_prefill_seq(q, k, v, alpha=a, b=b, w=w, initial_state=r.standard_normal((2, 2, 4, 3)))
    o2, S2 = od.dgda_prefill_seq(q, k, v, alpha=a, b=b, w=w, initial_state=np.zeros((2, 2, 4, 3)))
    np.testing.assert_allclose(o1, o2, atol=1e-12)
    np.testing.assert_allclose(S1, S2, atol=1e-12)


def test_zero_gates_freeze_state():
    q, k, v, a, b, w = _rand(1, 2, 7, 4, 3, 2)
    a[:] = 1.0
    b[:] = 0.0
    w[:] = 0.0
    S0 = np.random.default_rng(3).standard_normal((1, 2, 4, 3))
    o, S = od.dgda_prefill_seq(q, k, v, alpha=a, b=b, w=w, initial_state=S0)
    np.testing.assert_allclose(S, S0, atol=1e-12)
    np.testing.assert_allclose(o, np.einsum("bhtk,bhkv->bhtv", q, S0), atol=1e-12)


def test_single_token_prefill_equals_step():
    q, k, v, a, b, w = _rand(2, 3, 1, 6, 5, 4)
    S0 = np.random.default_rng(5).standard_normal((2, 3, 6, 5))
    o, S = od.dgda_prefill_seq(q, k, v, alpha=a, b=b, w=w, initial_state=S0)
    o2, S2 = od.dgda_step(q, k, v, alpha=a, b=b, w=w, state=S0)
    np.testing.assert_allclose(o[:, :, 0], o2, atol=1e-12)
    np.testing.assert_allclose(S, S2, atol=1e-12)


def test_chunk_chaining():
    q, k, v, a, b, w = _rand(1, 2, 30, 4, 4, 6)
    o, S = od.dgda_prefill_seq(q, k, v, alpha=a, b=b, w=w)
    sl = lambda x, s: x[:, :, s]
    o1, S1 = od.dgda_prefill_seq(*(sl(x, slice(0, 11)) for x in (q, k, v)), alpha=a[:, :, :11], b=b[:, :, :11],
                                 w=w[:, :, :11])
    o2, S2 = od.dgda_prefill_seq(*(sl(x, slice(11, 30)) for x in (q, k, v)), alpha=a[:, :, 11:], b=b[:, :, 11:],
                                 w=w[:, :, 11:], initial_state=S1)
    np.testing.assert_allclose(np.concatenate([o1, o2], axis=2), o, atol=1e-12)
    np.testing.assert_allclose(S2, S, atol=1e-12)


def test_brute_force_matrix_form():
    q, k, v, a, b, w = _rand(2, 2, 9, 5, 3, 7)
    S0 = np.random.default_rng(8).standard_normal((2, 2, 5, 3))
    o, S = od.dgda_prefill_seq(q, k, v, alpha=a, b=b, w=w, initial_state=S0)
    o2, S2 = od.dgda_prefill_dense(q, k, v, alpha=a, b=b, w=w, initial_state=S0)
    np.testing.assert_allclose(o, o2, atol=1e-11)
    np.testing.assert_allclose(S, S2, atol=1e-11)


@pytest.mark.parametrize("chunk", [1, 3, 16, 64])
def test_chunked_algorithm_is_chunk_size_independent(chunk):
    q, k, v, a, b, w = _rand(1, 2, 70, 8, 6, 10)
    S0 = np.random.default_rng(1).standard_normal((1, 2, 8, 6)) * 0.1
    o, S = od.dgda_prefill_seq(q, k, v, alpha=a, b=b, w=w, initial_state=S0)
    oc, Sc = od.dgda_prefill_chunked(q, k, v, alpha=a, b=b, w=w, chunk_size=chunk, initial_state=S0)
    np.testing.assert_allclose(oc, o, atol=1e-10)
    np.testing.assert_allclose(Sc, S, atol=1e-10)


def test_unit_lower_triangular_inverse_all_ones():
    """(I + strict-lower ones)^-1 is bidiagonal (reference test_dgda_precision.py:102-129)."""
    n = 16
    M = np.tril(np.ones((n, n)), 0)
    inv = np.eye(n) - np.eye(n, k=-1)
    np.testing.assert_allclose(np.linalg.solve(M, np.eye(n)), inv, atol=1e-12)


@pytest.mark.parametrize("gates", ["token", "channel"])
@pytest.mark.parametrize("L,chunk", [(1, 64), (100, 64), (130, 16), (64, 64)])
def test_c_chunked_oracle_matches_sequential(gates, L, chunk):
    B, H, dk, dv = 2, 3, 16, 12
    q, k, v, a, b, w = _rand(B, H, L, dk, dv, L)
    if gates == "token":
        a = np.repeat(a[..., :1], dk, -1)
        b = np.repeat(b[..., :1], dk, -1)
        w = np.repeat(w[..., :1], dv, -1)
    la = np.log(a)
    S0 = np.random.default_rng(2).standard_normal((B, H, dk, dv)).astype(np.float32) * 0.1
    f32 = lambda x: x.astype(np.float32).astype(np.float64)
    q, k, v, la, b, w = (f32(x) for x in (q, k, v, la, b, w))
    o, S = od.dgda_prefill_seq(q, k, v, alpha=np.exp(la), b=b, w=w, initial_state=S0)
    g = (lambda x: x[..., :1]) if gates == "token" else (lambda x: x)
    oc, Sc = dgda_c.dgda_prefill_chunked_c(q, k, v, g(la), g(b), g(w), initial_state=S0, chunk_size=chunk)
    np.testing.assert_allclose(oc, o, atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(Sc, S, atol=2e-5, rtol=2e-5)


# ----------------------------------------------------------------------------- layer prologue

def _pro_inputs(B=2, L=9, C=8, K=4, seed=0):
    rng = np.random.default_rng(seed)
    xs = [rng.standard_normal((B, L, C)) for _ in range(6)]
    ws = [rng.standard_normal((C, K)) * 0.5 for _ in range(3)]
    return xs, ws


def test_prologue_identity_and_shift_kernels():
    """Tap [0,0,0,1] is the identity (y = silu(x)); tap [1,0,0,0] reads three tokens back,
    through the carried history for the first three tokens."""
    xs, _ = _pro_inputs()
    B, L, C = xs[0].shape
    ident = np.zeros((C, 4)); ident[:, 3] = 1.0
    shift = np.zeros((C, 4)); shift[:, 0] = 1.0
    hist = [np.full((B, C, 3), 0.25 * (i + 1)) + np.arange(3) for i in range(3)]
    q, k, v, *_ , nh = od.layer_prologue(*xs, ident, ident, shift, hist=hist, n_heads=2)
    silu = lambda z: z / (1 + np.exp(-z))  # noqa: E731
    assert np.allclose(q, silu(xs[0]))
    exp_v = np.concatenate([hist[2].transpose(0, 2, 1), xs[2]], axis=1)[:, :L]
    assert np.allclose(v, silu(exp_v))
    for i in range(3):   # new history = last three conv inputs
        assert np.allclose(nh[i], xs[i][:, L - 3:].transpose(0, 2, 1))


def test_prologue_gate_closed_forms_and_unit_keys():
    xs, ws = _pro_inputs()
    xs[3][:] = 0.0
    xs[3][0, 0, 0] = 50.0           # softplus(50) = 50 -> clamped to -14
    xs[4][:] = 0.0
    q, k, v, la, al, b, w, _ = od.layer_prologue(*xs, *ws, n_heads=2)
    assert np.isclose(la[0, 0, 0], -14.0)
    assert np.allclose(la.ravel()[1:], -np.log(2.0))
    assert np.allclose(al, np.exp(la))
    assert np.allclose(b, 0.5)
    norms = np.sqrt((k.reshape(2, 9, 2, 4) ** 2).sum(-1))
    assert np.allclose(norms, 1.0, atol=1e-5)


def test_prologue_history_carry_equals_one_pass():
    xs, ws = _pro_inputs(L=12)
    full = od.layer_prologue(*xs, *ws, n_heads=2)
    first = od.layer_prologue(*[x[:, :5] for x in xs], *ws, n_heads=2)
    second = od.layer_prologue(*[x[:, 5:] for x in xs], *ws, hist=first[7], n_heads=2)
    for j in range(7):
        assert np.allclose(np.concatenate([first[j], second[j]], axis=1), full[j])
    for i in range(3):
        assert np.allclose(second[7][i], full[7][i])


def test_prologue_torch_reference_matches_oracle():
    """The dispatcher's torch prologue (the CPU path and the fallback) against the oracle."""
    import torch
    from maba_sparse.kernels import common as C
    xs, ws = _pro_inputs(B=2, L=11, C=16, seed=3)
    hist = [np.random.default_rng(i).standard_normal((2, 16, 3)) for i in range(3)]
    T = lambda a: torch.from_numpy(np.asarray(a))  # noqa: E731
    got = C.ref_dgda_prologue([T(x) for x in xs], [T(w).unsqueeze(1) for w in ws], [T(h) for h in hist],
                              n_heads=4, eps=1e-6)
    exp = od.layer_prologue(*xs, *ws, hist=hist, n_heads=4, eps=1e-6)
    for j in range(7):
        assert np.allclose(got[j].numpy(), exp[j], rtol=1e-10, atol=1e-12), j
    for i in range(3):
        assert np.allclose(got[7][i].numpy(), exp[7][i])
