"""The Scheme II planner (product host code) against the reference's recorded decisions.

- moduli sets at b = 54, 16 moduli requested (measure_logs/cool_oz2int8_{3520,7040,14080}.log:22)
  and the 15-modulus set at 128^3 (tools/validated/quick.csv:13);
- automatic width b, number of moduli and the one-pass error estimate at 4096^3, seed 7, for
  phi = 0 ... 16 (accuracy_logs/phi_sweep.log:122,266,410,554,698,842 and phi_sweep_05.log:122);
- closed-form invariants of every selection (coprimality, window inequality, int32 exactness).
"""
import math

import numpy as np
import pytest

import oztt_amd as oz

HEAD = [255, 254, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199]


@pytest.mark.parametrize("K,tail", [(3520, [37, 43]), (7040, [53, 61]), (14080, [37, 173])])
def test_moduli_records(K, tail):
    p = oz.choose_moduli_int8(K, 16, 54)
    assert p.ok and p.b == 54 and [p.m[i] for i in range(p.S)] == HEAD + tail


def test_moduli_quick_128():
    p = oz.choose_moduli_int8(128, 16, 54)
    assert p.ok and p.S == 15 and p.b == 54


@pytest.mark.parametrize("K", [32, 64, 1024, 4096, 8192, 16384, 65536, 133120])
@pytest.mark.parametrize("b_cap", [54, 60, 84, 100])
def test_selection_invariants(K, b_cap):
    p = oz.choose_moduli_int8(K, 24, b_cap)
    ms = [p.m[i] for i in range(p.S)]
    for i in range(len(ms)):
        for j in range(i + 1, len(ms)):
            assert math.gcd(ms[i], ms[j]) == 1
    if p.ok:
        M = math.prod(ms)
        assert M > 2 * K * 2 ** (2 * p.b)                    # the CRT window covers |C'| <= K 2^(2b)
        assert all(K * (m // 2) ** 2 <= 2 ** 31 - 1 for m in ms)  # int32-exact products
        assert p.b <= b_cap


PHI_RECORDS = [  # phi, auto b, moduli, recon1_pred of the research planner (two-pass forced), reference logs
    (0.0, 53, 15, -62.44), (0.5, 56, 16, -60.51), (1.0, 57, 16, -59.59), (2.0, 59, 16, -58.24),
    (4.0, 61, 17, -54.44), (8.0, 69, 19, -47.71), (16.0, 84, 23, -32.95)]
TABLE = [255, 254, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199, 197, 193, 191, 181, 179, 173, 167, 163,
         157, 151]


def research_int8_set(K, b_cap, wlog2):
    """The INT8 selection of the research planner that wrote the phi-sweep logs: the library's rules
    (moduli.hpp:719-769) with the CRT window log2 K replaced by a window measured from the input
    (experiments/src/ozaki2/ozaki2_autop.hpp:104-108). Test-side restatement; the library keeps log2 K."""
    ms, logM = [], 0.0
    for m in TABLE:
        ms.append(m)
        logM += math.log2(m)
    b = min(math.floor((logM - 1.0 - wlog2 - 1e-9) / 2.0), 100, b_cap)
    need = 2.0 * b + 1.0 + wlog2 + 1e-9
    while len(ms) > 2 and logM - math.log2(ms[-1]) >= need:
        logM -= math.log2(ms.pop())
    head = ms[:-2]
    base = sum(math.log2(x) for x in head)
    best, bp, bq, bcost = logM, ms[-2], ms[-1], 2
    over = lambda l: 1 if l - need > 0.25 else 0
    def better(c, l):
        if c != bcost:
            return c < bcost
        if over(l) != over(best):
            return over(l) < over(best)
        return l < best
    if logM > need:
        step = 2 if any(x % 2 == 0 for x in head) else 1
        cop = lambda v: all(math.gcd(v, x) == 1 for x in head)
        for p in range(3, 256, step):
            if not cop(p):
                continue
            lp = base + math.log2(p)
            if lp >= need and better(1, lp):
                best, bp, bq, bcost = lp, p, 0, 1
            for q in range(p + step, 256, step):
                if math.gcd(p, q) == 1 and cop(q):
                    lq = lp + math.log2(q)
                    if lq >= need and better(2, lq):
                        best, bp, bq, bcost = lq, p, q, 2
        ms = head + [bp] + ([bq] if bq else [])
    return ms, b


@pytest.mark.parametrize("phi,b,S,pred", [PHI_RECORDS[i] for i in (0, 1, 4, 6)])
def test_auto_precision_records(phi, b, S, pred):
    n = 4096
    a, bb = oz.eval_inputs(7, phi, n * n, n * n)
    p = oz.plan2_int8(a, bb, n, n, n, reconstruction=oz.Reconstruction.TwoPass)
    assert p.b == b and p.two_pass == 1 and p.nd == (5 if b > 80 else 4 if b > 60 else 3)
    # the library's window (log2 K) needs at least as many moduli as the research set, and the route
    # keeps it; the execution set covers the operands' own window (Cauchy-Schwarz on A', B'), which is
    # the research planner's measured window made rigorous, and needs as many moduli as its set
    lib = oz.choose_moduli_int8(n, 24, b)
    assert p.rS == lib.S and lib.S >= S
    assert (p.S_window or p.S) == lib.S and p.S == S
    # the statistics behind b reproduce the research planner's one-pass estimate to 0.01 bit
    r = math.sqrt(n)
    f = (1 + r / math.ldexp(p.wA, b)) * (1 + r / math.ldexp(p.wB, b))
    wlog2 = math.log2(p.wA * p.wB * max(f, 1.001))
    ms, b_r = research_int8_set(n, b, wlog2)
    assert b_r == b and len(ms) == S
    est = -70.0 + sum(math.log2(m) for m in ms) - 2.0 * b + 0.5 * (math.log2(p.TA) + math.log2(p.TB) - math.log2(p.nC))
    assert round(est, 2) == pred


def test_fixed_width_uses_sixteen_moduli():
    n = 4096
    a, bb = oz.eval_inputs(7, 0.0, 64 * n, n * 64)
    p = oz.plan2_int8(a, bb, 64, 64, n, reconstruction=oz.Reconstruction.OnePass, fixed_bits=54)
    assert p.b == 54 and p.S == 16 and p.two_pass == 0


def test_eval_inputs_match_reference_hashes():
    n = 4096
    a, b = oz.eval_inputs(7, 1.0, n * n, n * n)
    assert oz.eval_hash(a) == 0x108dbf997fae1816 and oz.eval_hash(b) == 0x292d509b232b2c21  # dgemm_ref.log:18


# ---- Scheme I ----------------------------------------------------------------------------------
# phi_sweep.log / phi_sweep_05.log (I-INT8, 4096^3, seed 7): the automatic p and the two model estimates
# at p (OZ_FP64 lines :47, :191, :335, :479, :623, :767 and phi_sweep_05.log:47).
OZ1_RECORDS = [  # phi, p, independent-sign bits, sampled bits
    (0.0, 7, 53.9, 53.8), (0.5, 8, 57.0, 54.2), (1.0, 8, 54.1, 53.9), (2.0, 9, 59.2, 56.2),
    (4.0, 9, 57.4, 55.2), (8.0, 9, 54.7, 53.9), (16.0, 11, 57.8, 58.1),
]


@pytest.mark.parametrize("phi,p,bi,bs", [OZ1_RECORDS[i] for i in (0, 2, 6)])
def test_scheme1_auto_p_matches_reference_records(phi, p, bi, bs):
    n = 4096
    a, b = oz.eval_inputs(7, phi, n * n, n * n)
    pl = oz.plan1(a, b, n, n, n)
    assert pl.p == p
    assert pl.pmax == 22  # ceil(160 / log2 254) + 1
    assert abs(pl.bits_indep - bi) <= 0.05 and abs(pl.bits_sampled - bs) <= 0.05
    assert (pl.Kc, pl.nkb, pl.pairloop, pl.pairwise, pl.fuse, pl.defer) == (n, 1, 0, 0, 0, 0)


def test_scheme1_issue_plans():
    """Closed forms of plan.hpp:130-206 and format.hpp:136-183 for the configurations of the BASELINE
    and the error paths."""
    z = np.zeros(64 * 64)
    # INT8, single K block up to (L+1) K 127^2 < 2^31
    pl = oz.plan1(z, z, 64, 64, 64, slices=8)
    assert (pl.p, pl.Kc, pl.nkb, pl.defer, pl.nsmall) == (8, 64, 1, 0, 0)
    # BF16 at C5's k = 65536 with 8 slices: pairwise issue, K blocks of 16384, int32 accumulation, deferred
    # reconstruction, no diagonal small enough to be read whole
    big = np.zeros(64 * 65536)
    pl = oz.plan1(big, big, 64, 64, 65536, slices=8, fmt=oz.Format.BF16)
    assert (pl.Kc, pl.nkb, pl.pairloop, pl.pairwise, pl.fuse, pl.defer, pl.nsmall) == (16384, 4, 0, 1, 1, 1, 0)
    # BF16 at 128^3 with 10 slices: the pair loop, all ten diagonals read whole (quick.csv:2)
    z128 = np.zeros(128 * 128)
    pl = oz.plan1(z128, z128, 128, 128, 128, slices=10, fmt=oz.Format.BF16)
    assert (pl.Kc, pl.nkb, pl.pairloop, pl.defer, pl.nsmall) == (128, 1, 1, 1, 10)


def test_scheme1_rejects_unsupported_plans():
    # INT8 would need two K blocks at k = 32768 with 8 slices (plan.hpp:187-195)
    z = np.zeros(64 * 32768)
    with pytest.raises(RuntimeError, match="K blocking"):
        oz.plan1(z, z, 64, 64, 32768, slices=8)
    # 16 slices of radix 254 overflow the FP32 exponent of the Horner evaluation (format.hpp:160-171)
    z = np.zeros(64 * 64)
    with pytest.raises(RuntimeError, match="overflow FP32"):
        oz.plan1(z, z, 64, 64, 64, slices=16)


# ---- Scheme II, FP8 route ----------------------------------------------------------------------
# cool_oz2fp8_{3520,7040,14080}.log:22 (fixed b = 54, 14 moduli requested): the set with its carrying
# methods (s sparse square, * square, k Karatsuba, w wide), matrix products, GEMM outputs after
# concatenation, and the concatenation bounds.
FP8_RECORDS = [
    (3520, "2401s 2209s 1849s 1681s 1521s 1369s 1024* 961* 841* 625* 289* 529*", 36, 24, 74,
     [4, 5, 7, 8, 9, 11, 18, 21, 24, 33, 74, 39]),
    (7040, "2401s 2209s 1849s 1681s 1521s 1369s 1024* 961* 841* 625* 529* 487k", 36, 25, 19,
     [2, 2, 3, 4, 4, 5, 9, 10, 12, 16, 19, 9]),
    (14080, "2401s 2209s 1849s 1681s 1521s 1369s 1024* 961* 841* 625* 529* 977w", 37, 28, 9,
     [1, 1, 1, 2, 2, 2, 4, 5, 6, 8, 9, 4]),
]
FP8_CODES = {0: "*", 1: "k", 2: "w", 4: "s"}


@pytest.mark.parametrize("K,mods,gemms,outs,maxg,maxg_m", FP8_RECORDS)
def test_fp8_moduli_records(K, mods, gemms, outs, maxg, maxg_m):
    p = oz.choose_moduli_fp8(K, 14, 54)
    assert p.ok and p.b == 54 and p.rsparse == 1 and p.rfold_first == 1
    got = " ".join(f"{p.rm[i]}{FP8_CODES[p.rmode[i]]}" for i in range(p.rS))
    assert got == mods
    assert (p.rnprod, p.rnout, p.rmaxg) == (gemms, outs, maxg)
    assert [p.rmaxg_m[i] for i in range(p.rS)] == maxg_m


def test_fp8_dense_digits_at_large_k():
    """K*32^2 + 2401 > 2^24 (K > 16381) returns to dense digits, the table up to 33^2 = 1089
    (moduli.hpp:724-731); every modulus then carries digits within 16."""
    p = oz.choose_moduli_fp8(16384, 24, 59)
    assert p.ok and p.b == 59 and p.rsparse == 0
    ms = [p.rm[i] for i in range(p.rS)]
    assert max(ms) <= 1089 and ms[:6] == [1089, 1024, 961, 841, 625, 529]
    assert all(math.gcd(x, y) == 1 for i, x in enumerate(ms) for y in ms[i + 1:])
    assert sum(math.log2(x) for x in ms) >= 2 * 59 + 1 + math.log2(16384)


# phi_sweep.log II-FP8 auto lines (4096^3, seed 7, two-pass forced): phi, b, moduli (CONFIG :110, :254, :398, :542)
FP8_PHI = [(0.0, 53, 12), (1.0, 57, 12), (2.0, 59, 12), (4.0, 61, 13)]


@pytest.mark.parametrize("phi,b,S", [FP8_PHI[i] for i in (0, 3)])
def test_fp8_auto_precision_records(phi, b, S):
    """The FP8 plan's width b equals the record; its set with the research planner's measured window has the
    recorded size; on the FP8 matrix cores the execution set is the route's FP8 set, or the FP8 set for the
    operands' own window (the research planner's window made rigorous) when that has fewer products."""
    n = 4096
    a, bb = oz.eval_inputs(7, phi, n * n, n * n)
    p = oz.plan2(a, bb, n, n, n, oz.Format.FP8, reconstruction=oz.Reconstruction.TwoPass)
    assert p.b == b and p.two_pass == 1
    r = math.sqrt(n)
    f = (1 + r / math.ldexp(p.wA, b)) * (1 + r / math.ldexp(p.wB, b))
    wlog2 = math.log2(p.wA * p.wB * max(f, 1.001))
    research = oz.choose_moduli_fp8(n, 24, b, wlog2)
    assert research.b == b and research.rS == S
    # by default the execution set is an FP8 set (its e4m3 digits on the FP8 matrix cores): the route's
    # with the full window; else the route's rules for the operands' window give a set of the research
    # set's size, and the execution set has at most its digit products (one-digit moduli included)
    full = oz.plan2(a, bb, n, n, n, oz.Format.FP8, reconstruction=oz.Reconstruction.TwoPass, full_window=True)
    assert full.fp8_digits and full.S_window == 0
    assert [full.m[i] for i in range(full.S)] == [p.rm[i] for i in range(p.rS)]
    assert math.log2(p.wA * p.wB) <= p.bound_log2 - 2 * b <= math.log2(n)
    own = oz.choose_moduli_fp8(n, 24, b, p.bound_log2 - 2 * b)
    assert own.b == b and own.rS == S
    assert p.fp8_digits and (p.S_window or p.S) == p.rS and p.nprod <= own.rnprod <= p.rnprod
    q = oz.plan2(a, bb, n, n, n, oz.Format.FP8, reconstruction=oz.Reconstruction.TwoPass,
                 transport=oz.Transport.Int8Residues)
    assert not q.fp8_digits and q.b == b and max(q.m[i] for i in range(q.S)) <= 255


@pytest.mark.parametrize("K,b", [(16384, 60), (4096, 54), (1024, 70)])
def test_fp8_carried_by_int8_residues(K, b):
    """Transport.Int8Residues: FP8 keeps the FP8 route's plan (width b, passes) and computes with an INT8 set
    of the same width: pairwise coprime moduli <= 255 whose window holds K 2^(2b) < M/2. Its int32 products
    are exact (K floor(m/2)^2 <= 2^31 - 1). The evaluation setting fp8_matrix_cores keeps the FP8 digits."""
    M = N = 64
    a, bb = oz.eval_inputs(4, 2.0, M * K, K * N)
    kw = dict(fixed_bits=b, max_moduli=24, reconstruction=oz.Reconstruction.OnePass)
    p = oz.plan2(a, bb, M, N, K, oz.Format.FP8, transport=oz.Transport.Int8Residues, **kw)
    f = oz.plan2(a, bb, M, N, K, oz.Format.FP8, transport=oz.Transport.Int8Residues, fp8_matrix_cores=True, **kw)
    assert oz.plan2(a, bb, M, N, K, oz.Format.FP8, **kw).fp8_digits
    i8 = oz.plan2(a, bb, M, N, K, oz.Format.INT8, fixed_bits=b, max_moduli=24,
                  reconstruction=oz.Reconstruction.OnePass)
    assert f.fp8_digits and not p.fp8_digits and not i8.fp8_digits
    # the route (what Info reports) is the FP8 route's either way
    assert p.rS == f.rS and [p.rm[i] for i in range(p.rS)] == [f.rm[i] for i in range(f.rS)]
    assert p.b == f.b == b and p.nd == f.nd and p.two_pass == f.two_pass
    # the execution set is the INT8 route's set at that width
    ms = [p.m[i] for i in range(p.S)]
    assert ms == [i8.m[i] for i in range(i8.S)] and i8.b == b
    assert max(ms) <= 255 and all(math.gcd(x, y) == 1 for i, x in enumerate(ms) for y in ms[i + 1:])
    assert sum(math.log2(x) for x in ms) >= 2 * b + 1 + math.log2(K)
    assert all(K * (x // 2) ** 2 <= 2**31 - 1 for x in ms)


def test_fp8_beyond_the_int8_width_keeps_its_digits():
    """At K = 4096, 24 moduli <= 255 hold a width of at most 85 bits and the FP8 route's up to 100; under
    Transport.Int8Residues a wider FP8 plan runs its own digits."""
    M = N = 64
    K = 4096
    a, bb = oz.eval_inputs(4, 2.0, M * K, K * N)
    assert oz.choose_moduli_int8(K, 24, 90).b == 85
    i8 = oz.Transport.Int8Residues
    p = oz.plan2(a, bb, M, N, K, oz.Format.FP8, fixed_bits=90, max_moduli=24, transport=i8)
    assert p.fp8_digits and p.b == 90 and (p.S_window or p.S) == p.rS
    p = oz.plan2(a, bb, M, N, K, oz.Format.FP8, fixed_bits=85, max_moduli=24, transport=i8)
    assert not p.fp8_digits and p.b == 85


def test_fp8_composition_coefficients_kat():
    """split.hpp:579: the radix-16 Karatsuba coefficients are (1-B, B^2-B, B) = (-15, 240, 16); squares use
    (1, q) with HL and LH concatenated. The device terms carry coefficient * y_s mod m_s."""
    M = N = 64
    K = 16384
    a, b = oz.eval_inputs(4, 2.0, M * K, K * N)
    dd, gd, crt, tm = oz.plan2_fp8_device(a, b, M, N, K, fixed_bits=60)
    S = dd.mo.S
    kar = [s for s in range(S) if dd.xmode[s] == 1]
    sq = [s for s in range(S) if dd.xmode[s] == 0]
    assert kar and sq
    for s in range(S):
        m, y = int(crt.m[s]), int(crt.y[s])
        outs = [gd.g[o] for o in range(gd.nout) if tm[o] == s]
        raw = sorted((g.coef * pow(y, -1, m)) % m for g in outs)
        if s in kar:
            assert raw == sorted(c % m for c in (-15, 240, 16)), (m, raw)
            assert all(g.npairs == 1 and g.a[0] - g.b[0] == 0 for g in outs)
        else:
            q = int(dd.q[s])
            assert q * q == m and raw == sorted([1, q % m]), (m, raw)
            assert sorted(g.npairs for g in outs) == [1, 2]


def test_fp8_rejects_k_beyond_exact_fp32():
    """moduli.hpp:472-500: K * 16^2 must stay within the exact FP32 integers; beyond, the plan fails with
    runtime_error naming the limit (no device work)."""
    M = N = 64
    K = 65600
    a = np.ones(M * K)
    b = np.ones(K * N)
    with pytest.raises(RuntimeError, match="too large for this format"):
        oz.plan2(a, b, M, N, K, oz.Format.FP8, fixed_bits=54)
    p = oz.plan2(a, b, M, N, K, oz.Format.INT8, fixed_bits=54)  # INT8 residues carry this K
    assert p.ok and p.b == 54


def test_moduli_limit_of_digit_routes():
    """Options.max_moduli bounds the format's own route (plan.hpp:281), as in the reference: a limit too
    small for the 53-bit window fails with runtime_error (tests/correctness.cpp:291-300 uses
    max_moduli = 2); a feasible limit is kept by the route's set; the evaluator's fixed width 54 with
    TF32's limit of 11 holds (evaluate.cpp:163-177)."""
    n = 128
    a, b = oz.eval_inputs(7, -1.0, n * n, n * n)
    for fmt in (oz.Format.BF16, oz.Format.FP16, oz.Format.TF32, oz.Format.BFP8, oz.Format.BFP4, oz.Format.BFP2):
        with pytest.raises(RuntimeError, match="max_moduli"):
            oz.plan2(a, b, n, n, n, fmt=fmt, max_moduli=2)
        p = oz.plan2(a, b, n, n, n, fmt=fmt, max_moduli=20)
        assert p.rS <= 20 and p.b >= 53 and not p.fp8_digits
    p = oz.plan2(a, b, n, n, n, fmt=oz.Format.TF32, max_moduli=11, fixed_bits=54)
    assert p.b == 54 and p.rS == 11


# Scheme II digit routes at b = 54 with the evaluator's moduli limits (evaluate.cpp:162: TF32 11, FP8 14,
# the others 24): (n, format, moduli, partial products) of tools/validated/quick.csv:3-17 (n = 128) and
# all.csv:3-49 (n = 3520, 7040, 14080; the table suite, m = n = k).
ROUTE_RECORDS = [(n, f, mod, pp) for n, rows in {
    128: [("BF16", 12, 30), ("FP16", 11, 31), ("TF32", 11, 33), ("BFP8", 12, 30), ("FP8", 12, 36), ("BFP4", 14, 65),
          ("BFP2", 18, 317)],
    3520: [("BF16", 11, 32), ("FP16", 11, 32), ("TF32", 11, 33), ("BFP8", 11, 32), ("FP8", 12, 36), ("BFP4", 15, 66),
           ("BFP2", 18, 336)],
    7040: [("BF16", 14, 30), ("FP16", 14, 30), ("TF32", 11, 33), ("BFP8", 14, 30), ("FP8", 12, 36), ("BFP4", 16, 62),
           ("BFP2", 19, 331)],
    14080: [("BF16", 14, 30), ("FP16", 14, 30), ("TF32", 11, 33), ("BFP8", 14, 30), ("FP8", 12, 37), ("BFP4", 17, 58),
            ("BFP2", 20, 329)],
}.items() for f, mod, pp in rows]
EVAL_LIMIT = {"TF32": 11, "FP8": 14}


@pytest.mark.parametrize("n,fmt,mod,pp", ROUTE_RECORDS)
def test_digit_route_records(n, fmt, mod, pp):
    """The route's set (the stage-time model's for BF16/FP16/BFP8/BFP4/BFP2, the table's for TF32 and FP8)
    has the recorded number of moduli and digit products, covers the window of b = 54 and is pairwise
    coprime."""
    f = oz.Format[fmt]
    r = oz.choose_moduli_route(f, n, n, n, EVAL_LIMIT.get(fmt, 24), 54)
    ms = [r.rm[i] for i in range(r.rS)]
    assert r.ok and r.b == 54 and (r.rS, r.rnprod) == (mod, pp), ms
    assert bool(r.rmodel_set) == (fmt not in ("TF32", "FP8"))
    assert all(math.gcd(x, y) == 1 for i, x in enumerate(ms) for y in ms[i + 1:])
    assert sum(math.log2(x) for x in ms) >= 2 * 54 + 1 + math.log2(n)


@pytest.mark.parametrize("b,mod,pp", [(56, 14, 32), (58, 14, 34), (60, 14, 35), (65, 14, 39), (76, 16, 46)])
def test_digit_route_phi_records(b, mod, pp):
    """BFP8 with automatic width at 14080^3, phi = 0.5, 1, 2, 4, 8 (all.csv:51-64): the stage-time model's
    set for the recorded width b (at most 24 moduli) has the recorded moduli and digit products."""
    r = oz.choose_moduli_route(oz.Format.BFP8, 14080, 14080, 14080, 24, b)
    assert r.ok and r.b == b and (r.rS, r.rnprod) == (mod, pp)


# quick.csv:3-17 Scheme II output hashes of the digit routes (128^3, uniform seed 7, b = 54, one pass)
ROUTE_HASHES = {"BF16": 0x13ABE4AC7F292F42, "FP16": 0x1811CF560959E61D, "TF32": 0x9A8F2780D4B9976B,
                "BFP8": 0x13ABE4AC7F292F42, "BFP4": 0x4AD3B42022EA6AD9, "BFP2": 0xC168D203062C72EF}


@pytest.mark.parametrize("fmt", list(ROUTE_HASHES))
def test_digit_route_reference_hashes(oracle, fmt):
    """The reference's published output of each digit route at 128^3 follows from the planner's set: the
    exact residues of A'B' modulo the route's moduli (oracle residues of A' and B', int64 products)
    through the oracle's restatement of the reference reconstruction (recon_crt.cpp) hash to the record.
    The hash depends on every modulus of the set, so it pins the stage-time model's choice; Info reports
    this set while the device computes with INT8 residues at the same width."""
    n = 128
    a, b = oz.eval_inputs(7, -1.0, n * n, n * n)
    f = oz.Format[fmt]
    p = oz.plan2(a, b, n, n, n, f, max_moduli=EVAL_LIMIT.get(fmt, 24), fixed_bits=54,
                 reconstruction=oz.Reconstruction.OnePass)
    assert p.b == 54 and not p.fp8_digits and p.two_pass == 0
    ms = [p.rm[i] for i in range(p.rS)]
    A, B = a.reshape(n, n), b.reshape(n, n)
    shift = 54 - 40
    dA, _ = oracle.scale(A, n, n, 0, 1, shift)
    dB, _ = oracle.scale(B, n, n, 1, 1, shift)
    ra = oracle.residues(A, n, n, 0, dA, 3, ms).astype(np.int64)
    rb = oracle.residues(B, n, n, 1, dB, 3, ms).astype(np.int64)
    C = np.empty((len(ms), n, n), dtype=np.int32)
    for s, m in enumerate(ms):
        r = (ra[s] @ rb[s]) % m
        C[s] = np.where(r > m // 2, r - m, r)
    assert oracle.hash(oracle.crt_ref(C, n, n, ms, 54, 3, 0, dA, dB)) == ROUTE_HASHES[fmt]


def test_digit_route_beyond_the_int8_width_keeps_its_width_on_fp8_digits():
    """BFP8's route holds b = 90 at K = 4096 (17 moduli up to 4096), 24 INT8 moduli at most 85 bits: the call
    keeps b = 90 and carries it with the FP8 route's e4m3 digits at that width, and Info reports BFP8's
    route. A width that neither transport holds is refused with runtime_error, never lowered."""
    M = N = 64
    K = 4096
    a, b = oz.eval_inputs(4, 2.0, M * K, K * N)
    r = oz.choose_moduli_route(oz.Format.BFP8, M, N, K, 24, 90)
    assert r.ok and r.b == 90 and r.rS == 17
    p = oz.plan2(a, b, M, N, K, oz.Format.BFP8, fixed_bits=90, max_moduli=24)
    assert p.b == 90 and p.fp8_digits and p.rS == 17
    f8 = oz.plan2(a, b, M, N, K, oz.Format.FP8, fixed_bits=90, max_moduli=24)
    assert [p.m[i] for i in range(p.S)] == [f8.m[i] for i in range(f8.S)]
    # at K = 16384 BFP4's route holds 100 bits, 24 INT8 moduli 84 and the FP8 route 83: refused
    K = 16384
    a, b = oz.eval_inputs(4, 2.0, M * K, K * N)
    assert oz.choose_moduli_route(oz.Format.BFP4, M, N, K, 24, 100).b == 100
    assert oz.choose_moduli_int8(K, 24, 100).b == 84
    assert oz.choose_moduli_route(oz.Format.FP8, M, N, K, 24, 100).b == 83
    with pytest.raises(RuntimeError, match="width of 100 bits.*beyond what this device"):
        oz.plan2(a, b, M, N, K, oz.Format.BFP4, fixed_bits=100, max_moduli=24)


def test_digit_route_accumulation_limit_is_the_references():
    """The digit routes accumulate digit products in FP32 in the reference, which bounds K (moduli.hpp:472-500):
    TF32's digits up to 32 give K 32^2 > 2^24 at K = 20000, and the plan fails with the reference's
    runtime_error although this build's INT8 residues could carry that K (INT8 itself still runs)."""
    M = N = 64
    K = 20000
    a, b = oz.eval_inputs(1, 0.5, M * K, K * N)
    with pytest.raises(RuntimeError, match="too large for this format.*2\\^24"):
        oz.plan2(a, b, M, N, K, oz.Format.TF32)
    assert oz.plan2(a, b, M, N, K, oz.Format.INT8).ok
