"""Pins the CPU oracle (oracle/lr_oracle.c) before it is trusted.

The reference ships no golden vectors or unit tests for this path, so each
oracle function is checked against (a) an independent restatement in torch's
own CPU operators (oracle/torch_path.py: torch.round, torch._int_mm,
torch.rsqrt, torch.sigmoid, F.gelu are library routines, not a retyping of
the C), (b) brute force on small inputs, (c) closed forms, invariants and
hand-constructed special cases chosen so that a plausible mistake (wrong
rounding mode, dropped clamp, swapped scale order, FMA contraction, wrong
slot or index) fails at least one of them.
"""
import numpy as np
import pytest
import torch

from helpers import assert_bf16_close, assert_rope_close, bf16_randn, from_np, to_np
from oracle import bf16, reference as ref, torch_path as tp


def gen(seed):
    return torch.Generator().manual_seed(seed)


# --------------------------------------------------------------- bf16 ----
def test_bf16_conversion_matches_torch():
    x = torch.randn(1 << 16, generator=gen(1), dtype=torch.float32) * 1e3
    x[:8] = torch.tensor([0.0, -0.0, 1.0, -1.0, 3.3895e38, 1e-40, float("inf"), float("-inf")])
    ours = bf16.from_f32(x.numpy())
    theirs = x.bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.array_equal(bf16.to_f32(ours), x.bfloat16().float().numpy())


# ---------------------------------------------------------- quantizer ----
@pytest.mark.parametrize("rows,width", [(16, 5120), (7, 317), (3, 1), (5, 20480)])
def test_quantize_matches_torch_path(rows, width):
    x = bf16_randn((rows, width), gen(2), outliers=0.01)
    q, s = ref.quantize_rows(to_np(x))
    tq, ts = tp.quantize(x)
    assert np.array_equal(q, tq.numpy())
    assert np.array_equal(s, ts.reshape(-1).numpy())


def test_quantize_ties_round_to_even_and_clamp():
    # absmax 127 -> s = 1 exactly, so x/s is exact and the ties are real ties.
    row = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -127.0, 3.0]], np.float32)
    q, s = ref.quantize_rows(bf16.from_f32(row))
    assert s[0] == np.float32(1.0)
    assert q.tolist() == [[127, 0, 2, 2, 0, -2, -2, 126, -127, 3]]


def test_quantize_invariants():
    x = bf16_randn((64, 1024), gen(3), outliers=0.01)
    x[5] = 0                      # all-zero row
    x[6] = 1e-12                  # below the 1e-8 floor
    x[7, :] = 0
    x[7, 3] = -2.0                # a single non-zero element
    q, s = ref.quantize_rows(to_np(x))
    assert np.abs(q.astype(np.int32)).max() <= 127
    nz = np.abs(bf16.to_f32(to_np(x))).max(axis=1) >= 1e-8
    assert (np.abs(q[nz]).max(axis=1) == 127).all()
    assert s[5] == np.float32(1e-8) / np.float32(127) and not q[5].any() and not q[6].any()
    assert q[7, 3] == -127 and np.count_nonzero(q[7]) == 1
    qn, sn = ref.quantize_rows(to_np(-x))      # odd symmetry
    assert np.array_equal(qn, -q) and np.array_equal(sn, s)


def _division_mismatches(limit=200):
    """(absmax, x) bf16 pairs where rint(x * (1/s)) != rint(x / s)."""
    u = np.arange(0x3D80, 0x4380, dtype=np.uint16)         # bf16 in [2^-4, 2^8)
    vals = bf16.to_f32(u)
    xs = np.concatenate([vals, -vals]).astype(np.float32)
    found = []
    for m in vals:
        s = np.float32(m) / np.float32(127)
        x = xs[np.abs(xs) <= m]
        div = np.rint((x / s).astype(np.float32))
        mul = np.rint((x * (np.float32(1) / s)).astype(np.float32))
        for xi, d in zip(x[div != mul], div[div != mul]):
            found.append((m, xi, d))
            if len(found) == limit:
                return found
    return found


def test_quantize_uses_ieee_division_not_reciprocal():
    cases = _division_mismatches()
    assert len(cases) >= 100
    rows = np.array([[m, x] for m, x, _ in cases], np.float32)
    q, s = ref.quantize_rows(bf16.from_f32(rows))
    assert np.array_equal(q[:, 1], np.array([d for _, _, d in cases]).astype(np.int8))
    assert np.array_equal(q[:, 0], np.full(len(cases), 127, np.int8))


# --------------------------------------------------------------- GEMM ----
def test_int_mm_brute_force_and_torch():
    g = gen(5)
    a = torch.randint(-127, 128, (37, 200), dtype=torch.int8, generator=g)
    w = torch.randint(-127, 128, (45, 200), dtype=torch.int8, generator=g)
    c = ref.int_mm(a.numpy(), w.numpy())
    brute = a.numpy().astype(np.int64) @ w.numpy().astype(np.int64).T
    assert np.array_equal(c, brute)
    assert np.array_equal(c, tp.int_mm(a, w).numpy())
    # the same product through a [K, N] array of other strides
    assert np.array_equal(ref.int_mm(a.numpy(), b=np.ascontiguousarray(w.numpy().T)), brute)


def test_int_mm_extremes_do_not_overflow():
    k = 20480   # largest K of the path: 127^2 * 20480 < 2^31
    a = np.full((2, k), -127, np.int8)
    w = np.full((3, k), -127, np.int8)
    assert (ref.int_mm(a, w) == 127 * 127 * k).all()


def test_dequant_matches_torch_path():
    g = gen(6)
    acc = torch.randint(-(2**30), 2**30, (33, 65), dtype=torch.int32, generator=g)
    rs = torch.rand(33, 1, generator=g) / 127
    cs = torch.rand(1, 65, generator=g) * 4e-3 + 1e-3
    bias = (torch.randn(65, generator=g) * 0.02).bfloat16()
    for b in (None, bias):
        ours = ref.dequant(acc.numpy(), rs.numpy(), cs.numpy(), None if b is None else to_np(b))
        assert np.array_equal(ours, to_np(tp.epilogue(acc, rs, cs, b)))


def test_dequant_operation_order():
    # ((acc * rs) * cs) + bias differs from acc * (rs * cs) and from an FMA
    # for these values: a reordered or contracted oracle fails.
    acc = np.array([[16777217, 3, 123456789]], np.int32)
    rs = np.array([1.1], np.float32)
    cs = np.array([0.3, 0.7, 1e-7], np.float32)
    out = ref.dequant(acc, rs, cs)
    expect = bf16.from_f32(((acc.astype(np.float32) * rs[:, None]) * cs[None, :]).astype(np.float32))
    assert np.array_equal(out, expect)


# ----------------------------------------------------- gated residual ----
def test_gated_residual_matches_torch_path():
    g = gen(7)
    x = bf16_randn((2, 9, 64), g)
    u = bf16_randn((2, 9, 64), g)
    table = bf16_randn((3, 6 * 64), g, scale=0.1)
    idx = torch.tensor([0, 1, 2, 1, 0, 2, 2, 1, 0])
    for slot in (2, 5):
        ours = ref.gated_residual(to_np(x), to_np(u), to_np(table), idx.numpy(), slot)
        assert np.array_equal(ours, to_np(tp.gated_residual(x, u, table, idx, slot)))


def test_gated_residual_rounds_the_product_first():
    # x + bf16(g*u) vs bf16(x + g*u): 1 + (1 + 2^-8) * 2^-8 rounds differently.
    x = bf16.from_f32(np.array([[1.0]], np.float32))
    u = bf16.from_f32(np.array([[2.0 ** -8]], np.float32))
    table = bf16.from_f32(np.array([[0, 0, 1 + 2.0 ** -7, 0, 0, 0]], np.float32))
    out = bf16.to_f32(ref.gated_residual(x, u, table, np.array([0]), 2))
    assert out[0, 0] == np.float32(1.0 + 2.0 ** -7)


# ---------------------------------------------------------- RMS norm ----
def test_canonical_sum_is_exact_when_no_rounding_happens():
    # Squares of small integers sum exactly in fp32: the order cannot matter.
    v = (np.arange(5120) % 7 - 3).astype(np.float32)
    assert ref.canonical_sumsq(bf16.from_f32(v)) == float((v.astype(np.int64) ** 2).sum())


def test_canonical_sum_order():
    # 2^24 + 1 + 1 ... depends on the order; check the defined slot/tree order
    # on a row where chunk 0 carries a huge value and other chunks ones.
    v = np.zeros(2048 * 2, np.float32)
    v[0] = 4096.0              # square 2^24 in slot 0
    v[8::8] = 1.0              # one 1.0 in every other chunk
    got = ref.canonical_sumsq(bf16.from_f32(v))
    slots = np.zeros(256, np.float32)
    for j in range(v.size // 8):
        acc = slots[j % 256]
        for e in v[8 * j:8 * j + 8]:
            acc = np.float32(acc + np.float32(e * e))
        slots[j % 256] = acc
    h = 128
    while h:
        slots[:h] = (slots[:h] + slots[h:2 * h]).astype(np.float32)
        h //= 2
    assert got == float(slots[0])
    assert got != float(np.float32(2 ** 24) + np.float32(v.size // 8 - 1))  # a plain sequential sum


def test_rms_adaln_close_to_reference_semantics():
    g = gen(8)
    x = bf16_randn((2, 40, 5120), g, outliers=0.01)
    w = (1 + 0.05 * torch.randn(5120, generator=g)).bfloat16()
    table = bf16_randn((3, 6 * 5120), g, scale=0.1)
    idx = torch.randint(0, 3, (40,), generator=g)
    ours = ref.rms_adaln(to_np(x), to_np(w), to_np(table), idx.numpy(), 0, 1, 1e-6)
    theirs = to_np(tp.rms_adaln(x, w, table, idx, 0, 1, 1e-6))
    ulp = bf16.ulp_distance(ours, theirs)
    assert ulp.max() <= 1 and (ulp == 0).mean() > 0.99


def test_rms_adaln_closed_form():
    # constant row c: rms = |c|, so n = sign(c) * w; with scale = 0, shift = 0
    # and w = 1 the output is +-1 exactly.
    hidden = 1024
    x = np.full((3, hidden), 0, np.float32)
    x[0] = 3.0
    x[1] = -0.25
    x[2] = 7.0
    table = np.zeros((1, 6 * hidden), np.float32)
    out = bf16.to_f32(ref.rms_adaln(bf16.from_f32(x), bf16.from_f32(np.ones(hidden, np.float32)),
                                    bf16.from_f32(table), np.zeros(3, np.int64), 0, 1, 0.0))
    assert (out[0] == 1).all() and (out[1] == -1).all() and (out[2] == 1).all()
    # shift/scale slots land where they should: scale slot 1 = 1 doubles, shift slot 0 adds 0.5
    table[0, 1 * hidden:2 * hidden] = 1.0
    table[0, 0:hidden] = 0.5
    out = bf16.to_f32(ref.rms_adaln(bf16.from_f32(x), bf16.from_f32(np.ones(hidden, np.float32)),
                                    bf16.from_f32(table), np.zeros(3, np.int64), 0, 1, 0.0))
    assert (out[0] == 2.5).all() and (out[1] == -1.5).all()


def test_rms_adaln_quant_is_quantizer_of_rms_adaln():
    g = gen(9)
    x = bf16_randn((1, 33, 640), g)
    w = (1 + 0.05 * torch.randn(640, generator=g)).bfloat16()
    table = bf16_randn((2, 6 * 640), g, scale=0.1)
    idx = torch.arange(33) % 2
    y = ref.rms_adaln(to_np(x), to_np(w), to_np(table), idx.numpy(), 3, 4, 1e-6)
    q, s = ref.rms_adaln_quant(to_np(x), to_np(w), to_np(table), idx.numpy(), 3, 4, 1e-6)
    q2, s2 = ref.quantize_rows(y.reshape(-1, 640))
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_residual_rms_quant_equals_two_step():
    # The reference's own exactness probe (script/precompile.py:65-77):
    # residual_rms_quant == _gated_residual(., 2) then _rms_adaln_quant_int8(., 3, 4)
    g = gen(10)
    x = bf16_randn((1, 32, 5376), g)
    u = bf16_randn((1, 32, 5376), g)
    table = bf16_randn((2, 6 * 5376), g)
    idx = torch.arange(32) % 2
    w = np.ones(5376, np.uint16) * 0x3F80
    r, q, s = ref.residual_rms_quant(to_np(x), to_np(u), w, to_np(table), idx.numpy(), 1e-5)
    r2 = ref.gated_residual(to_np(x), to_np(u), to_np(table), idx.numpy(), 2)
    q2, s2 = ref.rms_adaln_quant(r2, w, to_np(table), idx.numpy(), 3, 4, 1e-5)
    assert np.array_equal(r, r2) and np.array_equal(q, q2) and np.array_equal(s, s2)


# --------------------------------------------------------- activations ----
def test_gelu_tanh_against_torch():
    x = torch.linspace(-12, 12, 20001).bfloat16()
    ours = ref.gelu_tanh(to_np(x))
    theirs = to_np(tp.gelu_tanh(x))
    # torch evaluates 1 + tanh(u) in fp32, which cancels in the negative tail
    # (0 below x = -7, a few % off near |y| ~ 1e-6); the closed form does not.
    # Ulp-compare where |y| > 1e-4, absolute error below.
    assert_bf16_close(ours, theirs, frac_exact=0.99, atol=1e-4)
    z = bf16.to_f32(ref.gelu_tanh(bf16.from_f32(np.array([0.0, 30.0, -30.0], np.float32))))
    assert z[0] == 0 and z[1] == 30 and z[2] == 0


def test_swiglu_against_torch():
    g = gen(11)
    p = bf16_randn((17, 2 * 96), g, scale=3.0)
    ours = ref.swiglu(to_np(p))
    ulp = bf16.ulp_distance(ours, to_np(tp.swiglu(p)))
    assert ulp.max() <= 1 and (ulp == 0).mean() > 0.99
    q, s = ref.swiglu_quant(to_np(p))
    q2, s2 = ref.quantize_rows(ours)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


# ------------------------------------------------------- golden fixtures ----
def test_golden_fixtures_reproduce():
    import golden_check
    golden_check.check_all(ref)


# ------------------------------------------------------ QK norm + RoPE ----
def _qk_inputs(seed, batch=2, tokens=37, heads=3, dim=128, rot=128):
    g = gen(seed)
    q = bf16_randn((batch, tokens, heads, dim), g, outliers=0.01)
    k = bf16_randn((batch, tokens, heads, dim), g)
    qw = (1 + 0.1 * torch.randn(dim, generator=g)).bfloat16()
    kw = (1 + 0.1 * torch.randn(dim, generator=g)).bfloat16()
    phase = torch.randn(tokens, rot, generator=g) * 3
    return q, k, qw, kw, phase.cos(), phase.sin()


@pytest.mark.parametrize("dim,rot", [(128, 128), (128, 16), (128, 64), (64, 64), (64, 32), (32, 16), (128, 0),
                                     (128, 48), (128, 112), (64, 48)])
def test_qk_norm_rope_close_to_reference_semantics(dim, rot):
    q, k, qw, kw, cos, sin = _qk_inputs(30 + dim + rot, dim=dim, rot=rot)
    ours = ref.qk_norm_rope(to_np(q), to_np(k), to_np(qw), to_np(kw), cos.numpy(), sin.numpy(), 1e-6)
    theirs = tp.qk_norm_rope(q, k, qw, kw, cos, sin, 1e-6)
    for o, t in zip(ours, theirs):
        assert_rope_close(o, to_np(t), rot)


def test_qk_norm_rope_closed_forms():
    dim, tokens = 128, 4
    c = np.where(np.arange(tokens * 2 * dim) % 3 == 0, -0.25, 4.0).astype(np.float32)
    x = np.repeat(c.reshape(tokens, 2, dim)[:, :, :1], dim, axis=2)[None]  # constant rows of +-2^k
    x16 = bf16.from_f32(x)
    ones = bf16.from_f32(np.ones(dim, np.float32))
    # cos = 1, sin = 0: out = n = sign(row) exactly (rstd = 1/|c| is exact for powers of two)
    qo, ko = ref.qk_norm_rope(x16, x16, ones, ones, np.ones((tokens, dim), np.float32),
                              np.zeros((tokens, dim), np.float32), 0.0)
    assert np.array_equal(bf16.to_f32(qo), np.sign(x)) and np.array_equal(qo, ko)
    # cos = 0, sin = 1 (a quarter turn): out[:h] = -n[h:], out[h:] = n[:h]
    g = gen(5)
    y = to_np(bf16_randn((1, tokens, 2, dim), g))
    w = to_np((1 + 0.1 * torch.randn(dim, generator=g)).bfloat16())
    n, _ = ref.qk_norm_rope(y, y, w, w, np.ones((tokens, dim), np.float32), np.zeros((tokens, dim), np.float32), 1e-6)
    r, _ = ref.qk_norm_rope(y, y, w, w, np.zeros((tokens, dim), np.float32), np.ones((tokens, dim), np.float32), 1e-6)
    nf, rf = bf16.to_f32(n), bf16.to_f32(r)
    assert np.array_equal(rf[..., :64], -nf[..., 64:]) and np.array_equal(rf[..., 64:], nf[..., :64])
    # partial rotary: dimensions past rotary_dim are the normalized row unchanged
    p, _ = ref.qk_norm_rope(y, y, w, w, np.cos(np.ones((tokens, 16), np.float32)),
                            np.sin(np.ones((tokens, 16), np.float32)), 1e-6)
    assert np.array_equal(p[..., 16:], n[..., 16:]) and not np.array_equal(p[..., :16], n[..., :16])
    # no rotary: the normalized row
    z, _ = ref.qk_norm_rope(y, y, w, w, np.zeros((tokens, 0), np.float32), np.zeros((tokens, 0), np.float32), 1e-6)
    assert np.array_equal(z, n)


@pytest.mark.parametrize("dim", [128, 64, 32])
def test_qk_sum_is_exact_when_no_rounding_happens(dim):
    v = (np.arange(dim) % 9 - 4).astype(np.float32)
    assert ref.qk_sumsq(bf16.from_f32(v)) == float((v.astype(np.int64) ** 2).sum())


@pytest.mark.parametrize("dim,ones,expect", [
    # A square of 2^24 at element 0 absorbs a lone 1 (2^24 + 1 ties to even),
    # but not a 2 formed by two 1s that meet first. The reference's ordered
    # reduction (model/kernels.py:333-344) pairs element i with i + 16 first
    # inside a 32-element chunk, then i + 8, ..., i + 1:
    (128, (1, 17), 2.0 ** 24 + 2),    # 1 and 17 meet at the first step
    (128, (2, 3), 2.0 ** 24),         # 2 and 3 only at the last; absorbed one by one
    (128, (1, 9), 2.0 ** 24 + 2),     # 1 and 9 meet at the second step
    # chunk sums (s0, s1, s2, s3) combine as (s0 + s2) + (s1 + s3):
    (128, (32, 96), 2.0 ** 24 + 2),   # s1 + s3 = 2 before meeting s0
    (128, (32, 64), 2.0 ** 24),       # s2 joins s0 alone, then s1
    (64, (2, 3), 2.0 ** 24),
    (64, (1, 33), 2.0 ** 24),         # chunks first: a flat 64-wide tree would pair 1 with 33
    (32, (4, 20), 2.0 ** 24 + 2),
    (32, (4, 5), 2.0 ** 24),
])
def test_qk_sum_order(dim, ones, expect):
    v = np.zeros(dim, np.float32)
    v[0] = 4096.0
    v[list(ones)] = 1.0
    got = ref.qk_sumsq(bf16.from_f32(v))
    assert got == expect
