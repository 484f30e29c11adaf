"""The C-ABI boundary on the CPU: the library loads, exports every symbol that
``include/maba_hip.h`` declares, and its host-side validation and workspace
sizing behave as documented.  No call here launches GPU work: every entry point
exercised returns before its first HIP call.
"""
import ctypes
import os
import re

import pytest

from maba_sparse import _native as N

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "maba_hip.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)      # drop comments
    text = re.sub(r"//[^\n]*", "", text)
    return set(re.findall(r"\b(maba_hip_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(N.LIB_PATH):
        pytest.skip("libmaba_hip.so not built (run __graft_entry__.build())")
    return N.load()


def test_header_matches_binding_table():
    declared = _declared_symbols()
    assert declared, "no declarations parsed"
    assert declared == set(N.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(N.LIB_PATH)
    for name in sorted(_declared_symbols()):
        assert hasattr(raw, name), f"{name} declared in maba_hip.h but not exported"


def test_abi_version(lib):
    assert lib.maba_hip_abi_version() == 1


def _t(shape, dtype=N.MABA_BF16, strides=None, data=0x10000):
    """A descriptor that is never dereferenced (validation-only calls)."""
    t = N.MabaTensor()
    t.data = data
    t.dtype = dtype
    t.ndim = len(shape)
    if strides is None:
        strides, acc = [], 1
        for s in reversed(shape):
            strides.insert(0, acc)
            acc *= s
    for i, (s, st) in enumerate(zip(shape, strides)):
        t.shape[i] = s
        t.stride[i] = st
    return ctypes.byref(t)


def test_prefill_rejects_bad_rank_with_message(lib):
    q = _t([2, 3, 4])
    rc = lib.maba_hip_dgda_prefill(q, q, q, None, q, q, q, None, q, q, 64, None, 0, None)
    assert rc == N.MABA_ERR_INVALID
    assert b"q must be [B,H,L,dk]" in lib.maba_hip_last_error()


def test_prefill_requires_a_decay_gate(lib):
    B, H, L, d = 1, 2, 8, 64
    q = _t([B, H, L, d])
    s = _t([B, H, d, d], N.MABA_F32)
    rc = lib.maba_hip_dgda_prefill(q, q, q, None, None, q, q, None, q, s, 64, None, 0, None)
    assert rc == N.MABA_ERR_INVALID
    assert b"alpha or log_alpha" in lib.maba_hip_last_error()


def test_prefill_shape_mismatch(lib):
    q = _t([1, 2, 8, 64])
    k = _t([1, 2, 9, 64])
    s = _t([1, 2, 64, 64], N.MABA_F32)
    rc = lib.maba_hip_dgda_prefill(q, k, q, None, q, q, q, None, q, s, 64, None, 0, None)
    assert rc == N.MABA_ERR_INVALID


def _slot_geometry(BH, nch, cus=256, min_u=16):
    """Chunks per slot U and segments per sequence: the B*H*nch chunks in (b,h)-major
    order are cut into slots of U = max(min_u, ceil(total / (2 * CUs))) chunks; a
    sequence that fits one slot is never cut."""
    U = max(min_u, -(-BH * nch // (2 * cus)))
    if nch <= U:
        return nch, 1
    return U, -(-(nch - 1) // U) + 1


def test_prefill_workspace_size_at_baseline_shape(lib):
    """B=4, H=10, T=32768 (512 chunks per head): slots of 40 chunks, so up to 14
    segments per head, each carrying a [64, 128] fp32 aggregate and an int32 chunk
    count.  No GPU here: the library assumes 256 CUs."""
    B, H, T, d = 4, 10, 32768, 64
    q = _t([B, H, T, d])
    gate = _t([B, H, T, d], N.MABA_F32, strides=[H * T, T, 1, 0])   # per-token, stride-0 channels
    n = lib.maba_hip_dgda_prefill_workspace_size(q, q, gate, gate)
    U, nseg = _slot_geometry(B * H, T // 64)
    assert (U, nseg) == (40, 14)
    assert n == B * H * nseg * (64 * 128 * 4 + 4)   # + one chunk count per segment
    short = _t([B, H, 1024, d])                               # 16 chunks: one slot per head, no workspace
    sgate = _t([B, H, 1024, d], N.MABA_F32, strides=[H * 1024, 1024, 1, 0])
    assert lib.maba_hip_dgda_prefill_workspace_size(short, short, sgate, sgate) == 16
    # per-channel gates: the sub-chunk path, slots of U sub-chunks of 16 tokens (160 at this shape)
    per_channel = _t([B, H, T, d], N.MABA_F32)
    U, nseg = _slot_geometry(B * H, T // 16, min_u=64)
    assert (U, nseg) == (160, 14)
    assert lib.maba_hip_dgda_prefill_workspace_size(q, q, per_channel, gate) == B * H * nseg * (64 * 128 * 4 + 4)
    # d_k = d_v = 32: the sub-chunk path with 32 x 64 segment maps
    q32 = _t([B, H, T, 32])
    pc32 = _t([B, H, T, 32], N.MABA_F32)
    assert lib.maba_hip_dgda_prefill_workspace_size(q32, q32, pc32, pc32) == B * H * nseg * (32 * 64 * 4 + 4)
    # d_k = 128, d_v = 128: two calls over the value halves share 128 x (64 + 128) maps
    q128 = _t([B, H, T, 128])
    pc128 = _t([B, H, T, 128], N.MABA_F32)
    assert lib.maba_hip_dgda_prefill_workspace_size(q128, q128, pc128, pc128) == B * H * nseg * (128 * 192 * 4 + 4)
    # fp16 q with fp16 gates (one dtype, the reference's contract) also takes it
    qh = _t([B, H, T, 64], N.MABA_F16)
    gh = _t([B, H, T, 64], N.MABA_F16)
    assert lib.maba_hip_dgda_prefill_workspace_size(qh, qh, gh, gh) == B * H * nseg * (64 * 128 * 4 + 4)
    # head sizes outside {32, 64, 128} and bf16 gates with fp32 q take the sequential kernel
    q48 = _t([B, H, T, 48])
    assert lib.maba_hip_dgda_prefill_workspace_size(q48, q48, _t([B, H, T, 48], N.MABA_F32), _t([B, H, T, 48], N.MABA_F32)) == 0
    qf = _t([B, H, T, 64], N.MABA_F32)
    assert lib.maba_hip_dgda_prefill_workspace_size(qf, qf, _t([B, H, T, 64]), _t([B, H, T, 64])) == 0


def test_index_topk_decode_validation(lib):
    q = _t([2, 4, 128])
    c = _t([2, 100, 128])
    out = _t([2, 4, 32], N.MABA_I64)
    rc = lib.maba_hip_index_topk_decode(q, c, 0.1, 0, out, None, None, 0, None)
    assert rc == N.MABA_ERR_INVALID and b"top_k must be positive" in lib.maba_hip_last_error()
    # top_k > 64 takes the general sorted path, which holds at most 16,384 blocks per row; the
    # refusal comes before anything launches
    c_long = _t([2, 20000, 128])
    rc = lib.maba_hip_index_topk_decode(q, c_long, 0.1, 65, _t([2, 4, 65], N.MABA_I64), None, None, 0, None)
    assert rc == N.MABA_ERR_UNSUPPORTED and b"16384" in lib.maba_hip_last_error()
    rc = lib.maba_hip_index_topk_decode(q, c, 0.1, 32, _t([2, 4, 32], N.MABA_F32), None, None, 0, None)
    assert rc == N.MABA_ERR_DTYPE
    rc = lib.maba_hip_index_topk_decode(q, c, 0.1, 32, out, None, None, 0, None)
    assert rc == N.MABA_ERR_WORKSPACE


def test_index_topk_decode_workspace_covers_scores_and_tile_maxima(lib):
    B, Hq, nb = 8, 10, 15625
    tiles = (nb + 63) // 64
    n = lib.maba_hip_index_topk_decode_workspace_size(B, Hq, nb, 32)
    assert n >= B * Hq * tiles * 64 * 4 + B * Hq * tiles * 8


def test_maba_sa_decode_validation(lib):
    B, H, dc, L = 2, 4, 128, 1000
    q = _t([B, H, dc], N.MABA_F32)
    c = _t([B, L, dc])
    hca = _t([B, L // 64, dc])
    idx = _t([B, 3, 32], N.MABA_I64)      # neither 1 nor H index rows
    gate = _t([B, 3], N.MABA_F32)
    out = _t([B, H, dc], N.MABA_F32)
    rc = lib.maba_hip_maba_sa_decode(q, c, hca, idx, gate, L, 0.125, 128, 4, 64, 64, out, None, 0, None)
    assert rc == N.MABA_ERR_INVALID and b"idx must be [B,1|H,K]" in lib.maba_hip_last_error()
    idx = _t([B, 1, 32], N.MABA_I64)
    rc = lib.maba_hip_maba_sa_decode(q, c, hca, idx, gate, L + 1, 0.125, 128, 4, 64, 64, out, None, 0, None)
    assert rc == N.MABA_ERR_INVALID and b"L out of range" in lib.maba_hip_last_error()
    rc = lib.maba_hip_maba_sa_decode(q, c, hca, idx, gate, L, 0.125, 128, 4, 64, 64, out, None, 0, None)
    assert rc == N.MABA_ERR_WORKSPACE


def _arr(*descs):
    T = ctypes.POINTER(N.MabaTensor)
    return (T * len(descs))(*[d if d is not None else T() for d in descs])


def _p(shape, dtype=N.MABA_BF16, data=0x10000):
    t = N.MabaTensor()
    t.data, t.dtype, t.ndim = data, dtype, len(shape)
    acc = 1
    for i in reversed(range(len(shape))):
        t.shape[i], t.stride[i] = shape[i], acc
        acc *= shape[i]
    return ctypes.pointer(t)


def test_dgda_prologue_validation(lib):
    """Host checks of the prologue: 64-channel heads, one projection dtype, and a new
    conv history that does not alias the old one (each call returns before any launch)."""
    B, L, C = 2, 40, 640
    xs = _arr(*[_p([B, L, C]) for _ in range(6)])
    cw = _arr(*[_p([C, 1, 4], N.MABA_F32) for _ in range(3)])
    hist = [_p([B, C, 3], N.MABA_F32, data=0x20000 + 0x1000 * i) for i in range(3)]
    ys = _arr(*[_p([B, L, C]) for _ in range(3)], *[_p([B, L, C], N.MABA_F32) for _ in range(4)])
    fresh = _arr(*[_p([B, C, 3], N.MABA_F32, data=0x40000 + 0x1000 * i) for i in range(3)])
    aliased = _arr(_p([B, C, 3], N.MABA_F32, data=0x40000), hist[0], _p([B, C, 3], N.MABA_F32, data=0x48000))
    rc = lib.maba_hip_dgda_prologue(xs, cw, _arr(*hist), 1e-6, ys, aliased, None)
    assert rc == N.MABA_ERR_INVALID and b"must not alias" in lib.maba_hip_last_error()
    odd = _arr(*[_p([B, L, 100]) for _ in range(6)])
    rc = lib.maba_hip_dgda_prologue(odd, cw, None, 1e-6, ys, fresh, None)
    assert rc == N.MABA_ERR_UNSUPPORTED and b"64 * H" in lib.maba_hip_last_error()
    mixed = _arr(*[_p([B, L, C]) for _ in range(5)], _p([B, L, C], N.MABA_F32))
    rc = lib.maba_hip_dgda_prologue(mixed, cw, None, 1e-6, ys, fresh, None)
    assert rc == N.MABA_ERR_UNSUPPORTED and b"share one" in lib.maba_hip_last_error()
    bad_w = _arr(*[_p([C, 1, 3], N.MABA_F32) for _ in range(3)])
    rc = lib.maba_hip_dgda_prologue(xs, bad_w, None, 1e-6, ys, fresh, None)
    assert rc == N.MABA_ERR_INVALID


def test_check_maps_status_to_python_exceptions(lib):
    q = _t([2, 3, 4])
    rc = lib.maba_hip_dgda_prefill(q, q, q, None, q, q, q, None, q, q, 64, None, 0, None)
    with pytest.raises(ValueError, match="dgda_prefill"):
        N.check(rc, "dgda_prefill")
    rc = lib.maba_hip_index_topk_decode(_t([2, 4, 128]), _t([2, 20000, 128]), 0.1, 65,
                                        _t([2, 4, 65], N.MABA_I64), None, None, 0, None)
    with pytest.raises(NotImplementedError):
        N.check(rc, "index_topk_decode")
