"""GPU parity of each Scheme II stage against the CPU oracle, through the C ABI (include/oz_hip.h).

Bar: bit-exact (delta and flags of the scale stage, FP32 digits, int8 residues, int32 products, FP64
reconstruction). Inputs are seeded and cover the edge cases of each stage."""
import math

import numpy as np
import pytest

from oztt_amd.device import Device, crt_desc, from_blocks, moduli_desc, to_blocks
from tests.oracle_lib import assert_residues

pytestmark = pytest.mark.gpu

INT8_16 = [255, 254, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199, 47, 79]  # K=8192, b=54


def edge_matrix(rows, cols, rng):
    """Rows exercising the maxima rules: zero row, exact powers of two, dropped significand bits,
    the BF16 extremes, subnormal-only, huge, NaN, Inf; the rest random over 60 binades."""
    X = rng.uniform(-1, 1, (rows, cols)) * np.exp2(rng.integers(-30, 30, (rows, 1)))
    X[0] = 0.0
    X[1, :] = 0.5
    X[1, 3] = -1.0                       # exact power of two maximum
    X[2, 5] = 1.0 + 2.0 ** -40           # dropped bits below the BF16 significand
    X[3, 7] = float.fromhex("0x1.fep127")  # largest BF16
    X[4, :] = 0.0
    X[4, 2] = 2.0 ** -130                # nonzero maximum below 2^-126
    X[5, 1] = float.fromhex("0x1.ff8p127")  # above the largest BF16
    X[6, 9] = np.nan
    X[7, 4] = -np.inf
    X[8, :] = 2.0 ** -126                # smallest admissible maximum
    X[9, 0] = float.fromhex("0x1.fe00000000001p127")  # rounds up past the BF16 range
    return X


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("ceil_mode", [0, 1, 2])
def test_scale_matches_oracle(dev, oracle, mode, ceil_mode):
    rng = np.random.default_rng(100 + 3 * mode + ceil_mode)
    rows, cols = (70, 300) if mode == 0 else (300, 70)
    X = edge_matrix(rows, cols, rng) if mode == 0 else edge_matrix(cols, rows, rng).T.copy()
    shift = 14
    want_d, want_f = oracle.scale(X, rows, cols, mode, ceil_mode, shift)
    bx = dev.upload(X)
    n = rows if mode == 0 else cols
    bd = dev.alloc(4 * n)
    bf = dev.alloc(8)
    dev.fill_u32(bf, 0, 2)
    dev.scale(bx, rows, cols, cols, mode, ceil_mode, shift, bd, bf)
    got_d = dev.download(bd, np.int32, n)
    got_f = int(dev.download(bf, np.uint32, 1)[0])
    np.testing.assert_array_equal(got_d, want_d)
    assert got_f == want_f
    assert want_f == (6 if ceil_mode == 0 else 7)  # rounding down keeps 0x1.ff8p127 inside the BF16 range


def test_scale_large_column_reduction(dev, oracle):
    # many row chunks per column strip (atomic combination across workgroups)
    rng = np.random.default_rng(7)
    rows, cols = 4096, 192
    X = rng.standard_normal((rows, cols)) * np.exp2(rng.integers(-20, 20, (rows, cols)))
    want_d, want_f = oracle.scale(X, rows, cols, 1, 1, 14)
    bx = dev.upload(X)
    bd = dev.alloc(4 * cols)
    bf = dev.alloc(8)
    dev.fill_u32(bf, 0, 2)
    dev.scale(bx, rows, cols, cols, 1, 1, 14, bd, bf)
    np.testing.assert_array_equal(dev.download(bd, np.int32, cols), want_d)
    assert int(dev.download(bf, np.uint32, 1)[0]) == want_f == 0


def split_inputs(rows, cols, rng, phi):
    """Random operand with wide exponent spread plus crafted rounding-boundary elements."""
    X = (rng.uniform(0, 1, (rows, cols)) - 0.5) * np.exp(phi * rng.standard_normal((rows, cols)))
    X[0, :] = 0.0
    X[1, 0] = 1.0
    X[1, 1] = 2.0 ** -55 + 2.0 ** -80   # digits.h:44: with b = 54 and row maximum 1, A' = 0
    X[1, 2] = 2.0 ** -55                # exact half: ties to even
    X[1, 3] = 3 * 2.0 ** -55            # exact 1.5 ulp of A'
    X[1, 4] = -(2.0 ** -54) * 5 - 2.0 ** -55
    X[2, :] = rng.uniform(-1, 1, cols) * 2.0 ** -70   # far below the row maximum
    X[2, 0] = 1.0
    X[3, :] = np.ldexp(rng.integers(-2 ** 52, 2 ** 52, cols).astype(np.float64), -52)  # full significands
    # 90-120 binades below the row maximum: after scaling their low limbs fall below 2^-126 and flush
    X[4, :] = rng.uniform(-1, 1, cols) * np.exp2(-rng.integers(90, 121, cols).astype(np.float64))
    X[4, 0] = 1.0
    return X


@pytest.mark.parametrize("nd,b", [(3, 54), (3, 60), (4, 72), (5, 96)])
def test_digits_match_oracle(dev, oracle, nd, b):
    rng = np.random.default_rng(nd * 100 + b)
    rows, cols = 37, 129
    X = split_inputs(rows, cols, rng, 2.0)
    shift = b - 20 * (nd - 1)
    delta, _ = oracle.scale(X, rows, cols, 0, 1, shift)
    want = oracle.digits(X, rows, cols, 0, delta, nd)
    bx, bd = dev.upload(X), dev.upload(delta)
    bo = dev.alloc(4 * rows * cols * nd)
    dev.digits(bx, rows, cols, cols, 0, bd, nd, bo)
    got = dev.download(bo, np.float32, rows * cols * nd).reshape(rows, cols, nd)
    np.testing.assert_array_equal(got, want)  # values (a zero's sign may differ, it carries no value)
    if nd == 3 and b == 54:
        A1 = sum(float(want[1, 1, j]) * 2.0 ** (20 * (nd - 1 - j)) for j in range(nd))
        assert A1 == 0.0  # the documented example of the reference


def moduli_for(b, nd, K):
    from oztt_amd import choose_moduli_int8
    p = choose_moduli_int8(K, 24, b)
    return [p.m[i] for i in range(p.S)]


@pytest.mark.parametrize("layout", [0, 1, 2, 3])
@pytest.mark.parametrize("nd,b,phi", [(3, 54, 0.5), (3, 56, 2.0), (4, 70, 4.0), (5, 90, 1.0)])
def test_residues_match_oracle(dev, oracle, layout, nd, b, phi):
    """Layouts 0/2: A operand (rows of X = plane rows); 1/3: B operand (plane rows = columns of X).
    Layouts 2/3 are the OZ_BLOCK tiles of the GEMM, decoded on the host."""
    rng = np.random.default_rng(1000 + 10 * nd + layout)
    tran = layout in (1, 3)
    rows, cols = (200, 96) if tran else (96, 200)
    X = split_inputs(cols, rows, rng, phi).T.copy() if tran else split_inputs(rows, cols, rng, phi)
    mode = 1 if tran else 0
    shift = b - 20 * (nd - 1)
    moduli = moduli_for(b, nd, 4096)
    if 254 not in moduli:
        moduli = moduli + [254] if len(moduli) < 24 else moduli[:-1] + [254]
    delta, _ = oracle.scale(X, rows, cols, mode, 1, shift)
    want = oracle.residues(X, rows, cols, mode, delta, nd, moduli)  # [S][rows][cols]
    S = len(moduli)
    prow = (cols if tran else rows)
    prow = (prow + 63) // 64 * 64 + 64
    pld = ((rows if tran else cols) + 63) // 64 * 64 + 64
    pstride = prow * pld + 1024
    bx, bd = dev.upload(X), dev.upload(delta)
    bp = dev.alloc(S * pstride)
    dev.split_int8(bx, rows, cols, cols, mode, bd, moduli_desc(moduli, nd), bp, layout, prow, pld, pstride)
    got = dev.download(bp, np.int8, S * pstride).reshape(S, pstride)[:, :prow * pld]
    got = from_blocks(got, prow, pld) if layout >= 2 else got.reshape(S, prow, pld)
    if not tran:
        np.testing.assert_array_equal(got[:, :rows, :cols], want)
        assert not got[:, rows:, :].any() and not got[:, :, cols:].any()
    else:
        np.testing.assert_array_equal(got[:, :cols, :rows], want.transpose(0, 2, 1))
        assert not got[:, cols:, :].any() and not got[:, :, rows:].any()
    assert np.abs(want.astype(np.int32)).max() <= 127


@pytest.mark.parametrize("M,N,K,batch", [(256, 256, 128, 3), (512, 768, 384, 2), (256, 512, 1024, 1),
                                         (256, 256, 64, 2), (512, 256, 320, 1)])
def test_gemm_i8_exact(dev, M, N, K, batch):
    """Operands in OZ_BLOCK tiles; K/64 odd and K = 64 exercise the pipeline's tail."""
    rng = np.random.default_rng(M + N + K)
    A = rng.integers(-127, 128, (batch, M, K), dtype=np.int8)
    Bt = rng.integers(-127, 128, (batch, N, K), dtype=np.int8)
    A[0, 0, :] = 127
    Bt[0, 0, :] = 127       # largest positive sum
    A[0, 1, :] = -127       # largest negative sum
    bA, bB = dev.upload(to_blocks(A)), dev.upload(to_blocks(Bt))
    bC = dev.alloc(4 * batch * M * N)
    dev.gemm_i8(bA, bB, bC, M, N, K, batch, N, M * K, N * K, M * N)
    C = dev.download(bC, np.int32, batch * M * N).reshape(batch, M, N)
    for t in range(batch):
        want = A[t].astype(np.int64) @ Bt[t].astype(np.int64).T
        np.testing.assert_array_equal(C[t].astype(np.int64), want)


def test_gemm_i8_rejects_bad_shapes(dev):
    bA = dev.alloc(256 * 128)
    bC = dev.alloc(4 * 256 * 256)
    with pytest.raises(RuntimeError):
        dev.gemm_i8(bA, bA, bC, 256, 256, 96, 1, 256, 0, 0, 0)  # K not a multiple of 64
    with pytest.raises(RuntimeError):
        dev.gemm_i8(bA, bA, bC, 200, 256, 128, 1, 256, 0, 0, 0)  # M not a multiple of 256
    with pytest.raises(RuntimeError):
        dev.gemm_i8(bA, bA, bC, 256, 256, 128, 2, 256, 512, 512, 65536)  # batch stride not a multiple of 1 KB


def exact_double(cprime: int, e: int) -> float:
    """cprime * 2^e rounded to nearest-even, below 2^-1022 -> signed zero (the documented contract)."""
    if cprime == 0:
        return 0.0
    f = math.ldexp(float(cprime), e) if abs(cprime).bit_length() < 1020 else float(cprime) * 2.0 ** e
    if abs(f) < 2.0 ** -1022:
        return math.copysign(0.0, cprime)
    return f


@pytest.mark.parametrize("moduli,b,nd", [(INT8_16, 54, 3), ([255, 254, 253, 251, 247, 241, 239, 233, 229, 227, 223,
                                                              217, 211, 199, 197, 193, 191, 181, 179], 70, 4),
                                         ([251, 241, 239], 10, 3),
                                         # S M of 99 and 190 bits: 3 and 5 limbs of 40 bits in the digits kernel
                                         ([255, 254, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217], 40, 3),
                                         ([255, 254, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199, 197,
                                           193, 191, 181, 179, 173, 167, 163, 157, 151], 90, 5)])
def test_crt_exact(dev, oracle, moduli, b, nd):
    rng = np.random.default_rng(len(moduli) * 31 + b)
    Mprod = 1
    for m in moduli:
        Mprod *= m
    M, N = 3, 517
    n = M * N
    import random
    pyr = random.Random(int(b) * 7919 + len(moduli))
    half = (Mprod - 1) // 2
    vals = [pyr.randint(-half, half) >> pyr.randint(0, Mprod.bit_length() - 1) for _ in range(n)]
    vals[:8] = [0, 1, -1, half, -half, half - 1, -(half - 1), Mprod // 3]
    S = len(moduli)
    C = np.empty((S, M, N), dtype=np.int32)
    for idx, v in enumerate(vals):
        i, j = divmod(idx, N)
        for s, m in enumerate(moduli):
            r = v % m
            k = int(rng.integers(-(2 ** 31 - 1) // m + 1, (2 ** 31 - 1) // m - 1))
            C[s, i, j] = r + k * m  # any representative within int32
    dA = rng.integers(-5, 30, M).astype(np.int32)
    dB = rng.integers(-5, 30, N).astype(np.int32)
    shift = b - 20 * (nd - 1)
    bC, bdA, bdB = dev.upload(C), dev.upload(dA), dev.upload(dB)
    bo = dev.alloc(8 * n)
    dev.crt(bC, M, N, N, M * N, crt_desc(moduli, b, nd), bdA, bdB, bo, N)
    got = dev.download(bo, np.float64, n)
    want = np.array([exact_double(vals[idx], 2 * shift - int(dA[idx // N]) - int(dB[idx % N]) - 2 * b)
                     for idx in range(n)])
    np.testing.assert_array_equal(got.view(np.uint64), want.view(np.uint64))
    np.testing.assert_array_equal(got.view(np.uint64),
                                  oracle.crt_exact(C, M, N, moduli, b, nd, dA, dB).view(np.uint64))
    # the same from CRT digits k_s = (C_s mod m_s) y_s mod m_s (uint8 planes, row stride a multiple of 4);
    # the product kernels may store a digit 0 as m_s: half of the zero digits are given that way
    desc = crt_desc(moduli, b, nd)
    ldd = (N + 3) // 4 * 4 + 4
    D = np.zeros((S, M, ldd), dtype=np.uint8)
    for s, m in enumerate(moduli):
        k = C[s].astype(np.int64) % m * int(desc.y[s]) % m
        k = np.where((k == 0) & (rng.random(k.shape) < 0.5), m, k)
        D[s, :, :N] = k.astype(np.uint8)
    assert np.any(D == np.array(moduli, dtype=np.uint8)[:, None, None])
    bD = dev.upload(D)
    bo2 = dev.alloc(8 * n)
    dev.crt_digits(bD, M, N, ldd, M * ldd, desc, bdA, bdB, bo2, N)
    np.testing.assert_array_equal(dev.download(bo2, np.float64, n).view(np.uint64), want.view(np.uint64))


@pytest.mark.parametrize("moduli,b,nd", [(INT8_16 + [193], 56, 3),
                                         ([255, 254, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199, 197,
                                           193, 191, 181, 179, 173, 167, 163, 157, 151], 90, 5)])
def test_crt_rounding_ties(dev, moduli, b, nd):
    """C' exactly at, one above and one below a midpoint of the FP64 grid, with the rounding position in
    every 40-bit limb of the digits kernel (and the 32-bit limbs of the int32 kernel), both signs: the
    outputs of both CRT kernels are the correctly rounded C' (ties to even), against exact integers."""
    import random
    Mprod = 1
    for m in moduli:
        Mprod *= m
    half = (Mprod - 1) // 2
    pyr = random.Random(b * 131 + len(moduli))
    vals = []
    while len(vals) < 1500:
        n = pyr.randint(55, half.bit_length() - 1)
        base = pyr.getrandbits(n) | (1 << (n - 1))
        g = n - 53  # the rounding position
        base = (base >> g) << g
        mid = base + (1 << (g - 1))
        for v in (mid, mid + 1, mid - 1, base + (2 << g) + (1 << (g - 1))):
            if v <= half:
                vals.append(v if pyr.random() < 0.5 else -v)
    M, N = 3, len(vals) // 3
    vals = vals[:M * N]
    S = len(moduli)
    desc = crt_desc(moduli, b, nd)
    C = np.empty((S, M, N), dtype=np.int32)
    ldd = (N + 3) // 4 * 4 + 4
    D = np.zeros((S, M, ldd), dtype=np.uint8)
    for idx, v in enumerate(vals):
        i, j = divmod(idx, N)
        for s, m in enumerate(moduli):
            C[s, i, j] = v % m
            D[s, i, j] = (v % m) * int(desc.y[s]) % m
    shift = b - 20 * (nd - 1)
    # the exponent 2 shift - dA - dB - 2b is zero: the outputs are C' itself, rounded
    dA = np.full(M, shift - b, dtype=np.int32)
    dB = np.full(N, shift - b, dtype=np.int32)
    want = np.array([float(v) for v in vals])  # Python rounds an int to the nearest double, ties to even
    bC, bD, bdA, bdB = dev.upload(C), dev.upload(D), dev.upload(dA), dev.upload(dB)
    bo, bo2 = dev.alloc(8 * M * N), dev.alloc(8 * M * N)
    dev.crt(bC, M, N, N, M * N, desc, bdA, bdB, bo, N)
    dev.crt_digits(bD, M, N, ldd, M * ldd, desc, bdA, bdB, bo2, N)
    np.testing.assert_array_equal(dev.download(bo, np.float64, M * N).view(np.uint64), want.view(np.uint64))
    np.testing.assert_array_equal(dev.download(bo2, np.float64, M * N).view(np.uint64), want.view(np.uint64))
    for x in (bC, bD, bdA, bdB, bo, bo2):
        x.free()
    dev.bufs.clear()


@pytest.mark.parametrize("M,N,K,S", [(256, 512, 320, 17), (512, 256, 8192, 5)])
def test_gemm_digits_exact(dev, M, N, K, S):
    """oz2_gemm_digits: the products of oz_gemm_i8 reduced to CRT digits in the epilogue, bit-exact;
    K = 8192 with all-127 rows reaches the largest products the planner admits (K*127^2 < 2^31)."""
    moduli = INT8_16[:S] if S <= 16 else INT8_16 + [193]
    rng = np.random.default_rng(M * 3 + K)
    A = rng.integers(-127, 128, (S, M, K), dtype=np.int8)
    Bt = rng.integers(-127, 128, (S, N, K), dtype=np.int8)
    A[:, 0, :] = 127
    Bt[:, 0, :] = 127
    A[:, 1, :] = -127
    desc = crt_desc(moduli, 54, 3)
    bA, bB = dev.upload(to_blocks(A)), dev.upload(to_blocks(Bt))
    bD = dev.alloc(S * M * N)
    dev.gemm_digits(bA, bB, bD, M, N, K, S, N, M * K, N * K, M * N, desc)
    D = dev.download(bD, np.uint8, S * M * N).reshape(S, M, N)
    for s, m in enumerate(moduli):
        prod = (A[s].astype(np.float64) @ Bt[s].astype(np.float64).T).astype(np.int64)  # exact: |sum| < 2^53
        want = (prod % m) * int(desc.y[s]) % m
        assert_residues(D[s], want, m, f"modulus {m}")


def test_product_dispatch_timing(dev):
    """oz_time_products_begin/end: the product launches between them set the requested events from their
    own dispatches (the first launch the start, every launch the end), other launches do not consume the
    request, a request with no product launch reports so, and the timed products' results are those of
    untimed launches."""
    rng = np.random.default_rng(12)
    M = N = 512
    K, batch = 1024, 3
    A = rng.integers(-127, 128, (batch, M, K), dtype=np.int8)
    Bt = rng.integers(-127, 128, (batch, N, K), dtype=np.int8)
    bA, bB = dev.upload(to_blocks(A)), dev.upload(to_blocks(Bt))
    c1, c2 = dev.alloc(4 * batch * M * N), dev.alloc(4 * batch * M * N)
    args = (M, N, K, batch, N, M * K, N * K, M * N)
    dev.gemm_i8(bA, bB, c1, *args)
    # a request with no product launch in it (a fill only)
    dev.time_products_begin(30, 31)
    dev.fill_u32(c2, 0, batch * M * N)
    assert not dev.time_products_end()
    # two product launches under one request, events around the pair as markers
    dev.event_record(40)
    dev.time_products_begin(30, 31)
    dev.gemm_i8(bA, bB, c2, *args)
    dev.fill_u32(c2, 0, batch * M * N)
    dev.gemm_i8(bA, bB, c2, *args)
    assert dev.time_products_end()
    dev.event_record(41)
    dev.sync()
    t_products, t_markers = dev.elapsed_ms(30, 31), dev.elapsed_ms(40, 41)
    assert 0.0 < t_products <= t_markers
    np.testing.assert_array_equal(dev.download(c2, np.int32, batch * M * N), dev.download(c1, np.int32, batch * M * N))
    for x in (bA, bB, c1, c2):
        x.free()
    dev.bufs.clear()


def test_gemm_tile_pool_counts(dev):
    """The last eighth of every XCD's tiles is handed out through counters in the device handle, which
    each launch must leave at zero: launches of 1, 7, 9, 63, 65 and 1031 tiles back to back on one
    handle, int32 products (K/64 odd) and CRT digits (K/64 even), every output first filled with a
    sentinel, so a tile that no workgroup ran (or a stale counter) shows."""
    rng = np.random.default_rng(11)
    moduli = INT8_16 + [193]
    for M, N, batch in [(256, 256, 1), (256, 256, 7), (256, 768, 3), (768, 768, 7), (256, 1280, 13),
                        (256, 256, 1031)]:
        # digits: one batch per modulus, so at most the 17 moduli of the set (1031 tiles: int32 only)
        for digits in (False, True) if batch <= len(moduli) else (False,):
            K = 128 if digits else 192
            A = rng.integers(-127, 128, (batch, M, K), dtype=np.int8)
            Bt = rng.integers(-127, 128, (batch, N, K), dtype=np.int8)
            bA, bB = dev.upload(to_blocks(A)), dev.upload(to_blocks(Bt))
            esz = 1 if digits else 4
            out = dev.alloc(esz * batch * M * N)
            dev.fill_u32(out, 0xA5A5A5A5, esz * batch * M * N // 4)
            if digits:
                mods = moduli[:batch]
                desc = crt_desc(mods, 54, 3)
                dev.gemm_digits(bA, bB, out, M, N, K, batch, N, M * K, N * K, M * N, desc)
                got = dev.download(out, np.uint8, batch * M * N).reshape(batch, M, N)
            else:
                dev.gemm_i8(bA, bB, out, M, N, K, batch, N, M * K, N * K, M * N)
                got = dev.download(out, np.int32, batch * M * N).reshape(batch, M, N)
            for x in (bA, bB, out):
                x.free()
            dev.bufs.clear()
            prod = np.matmul(A.astype(np.float64), Bt.astype(np.float64).transpose(0, 2, 1)).astype(np.int64)
            for t in range(batch):
                if digits:
                    assert_residues(got[t], (prod[t] % mods[t]) * int(desc.y[t]), mods[t], f"{batch} tiles, batch {t}")
                else:
                    np.testing.assert_array_equal(got[t].astype(np.int64), prod[t], err_msg=f"{batch} tiles, batch {t}")


@pytest.mark.parametrize("M,N,K,S,digits", [(256, 256, 256, 300, False), (256, 512, 384, 150, False),
                                             (1024, 1024, 256, 20, True), (768, 1024, 384, 23, True)])
def test_gemm_tile_sequences(dev, M, N, K, S, digits):
    """More tiles than CUs (several generations of workgroups, the tile map over many batches), few
    K steps per tile (4 and 6), tile counts that are not a multiple of the CU or XCD count; int32
    products and CRT digits bit-exact."""
    rng = np.random.default_rng(M + 7 * S + K)
    A = rng.integers(-127, 128, (S, M, K), dtype=np.int8)
    Bt = rng.integers(-127, 128, (S, N, K), dtype=np.int8)
    A[:, 0, :] = 127
    Bt[:, 0, :] = 127
    A[:, 1, :] = -127
    bA, bB = dev.upload(to_blocks(A)), dev.upload(to_blocks(Bt))
    moduli = (INT8_16 + [193, 191, 181, 179, 173, 167, 163])[:S] if digits else None
    out = dev.alloc((1 if digits else 4) * S * M * N)
    if digits:
        desc = crt_desc(moduli, 54, 3)
        dev.gemm_digits(bA, bB, out, M, N, K, S, N, M * K, N * K, M * N, desc)
        got = dev.download(out, np.uint8, S * M * N).reshape(S, M, N)
    else:
        dev.gemm_i8(bA, bB, out, M, N, K, S, N, M * K, N * K, M * N)
        got = dev.download(out, np.int32, S * M * N).reshape(S, M, N)
    for x in (bA, bB, out):
        x.free()
    dev.bufs.clear()
    for t in range(S):
        prod = (A[t].astype(np.float64) @ Bt[t].astype(np.float64).T).astype(np.int64)  # exact: |sum| < 2^53
        if digits:
            assert_residues(got[t], (prod % moduli[t]) * int(desc.y[t]), moduli[t], f"batch {t}")
        else:
            np.testing.assert_array_equal(got[t].astype(np.int64), prod, err_msg=f"batch {t}")


def test_device_copy(dev):
    rng = np.random.default_rng(5)
    x = rng.integers(0, 2 ** 32, 4096 + 64, dtype=np.uint64).astype(np.uint32)
    src, dst = dev.upload(x), dev.alloc(4 * x.size)
    dev.copy(dst, src, 4 * x.size)
    np.testing.assert_array_equal(dev.download(dst, np.uint32, x.size), x)
    with pytest.raises(RuntimeError):
        dev.copy(dst, src, 20)  # not a multiple of 16


@pytest.mark.parametrize("layout", [2, 3])
@pytest.mark.parametrize("moduli", [[254, 128, 250, 249, 247, 3], [255, 253, 251, 2], [254]])
def test_residues_any_parity_of_moduli(dev, oracle, layout, moduli):
    """The blocked splitter takes odd moduli through byte dot products of A' and the one even modulus
    of a pairwise coprime set through the reference's sequence; a set with several even moduli (no
    plan has one) goes through the reference's sequence for all. Every case equals the oracle."""
    nd, b = 3, 56
    rng = np.random.default_rng(77 + layout + len(moduli))
    tran = layout == 3
    rows, cols = (160, 80) if tran else (80, 160)
    X = split_inputs(rows, cols, rng, 2.0)
    X[0, :4] = [254.0 * 2.0 ** -40, -127.0 * 2.0 ** -40, 0.0, 381.0 * 2.0 ** -40]  # values at +-m/2 of 254
    mode = 1 if tran else 0
    delta, _ = oracle.scale(X, rows, cols, mode, 1, b - 20 * (nd - 1))
    want = oracle.residues(X, rows, cols, mode, delta, nd, moduli)
    S = len(moduli)
    prow = ((cols if tran else rows) + 63) // 64 * 64
    pld = ((rows if tran else cols) + 63) // 64 * 64
    bx, bd = dev.upload(X), dev.upload(delta)
    bp = dev.alloc(S * prow * pld)
    dev.split_int8(bx, rows, cols, cols, mode, bd, moduli_desc(moduli, nd), bp, layout, prow, pld, prow * pld)
    got = from_blocks(dev.download(bp, np.int8, S * prow * pld).reshape(S, -1), prow, pld)
    for buf in (bx, bd, bp):
        buf.free()
    dev.bufs.clear()
    if tran:
        np.testing.assert_array_equal(got[:, :cols, :rows], want.transpose(0, 2, 1))
    else:
        np.testing.assert_array_equal(got[:, :rows, :cols], want)


@pytest.mark.parametrize("ceil_mode", [0, 1, 2])
@pytest.mark.parametrize("M,N,K", [(300, 200, 1000), (64, 1100, 77), (1, 1, 1), (2048, 40, 4096)])
def test_scale_pair_matches_oracle(dev, oracle, ceil_mode, M, N, K):
    """oz_scale_pair_f64: A's rows and B's columns in one launch, with leading dimensions beyond the
    extents, equal to the oracle's scale of each operand; flags 0 for finite in-range inputs."""
    rng = np.random.default_rng(M + N + K + ceil_mode)
    lda, ldb = K + 3, N + 5
    A = np.zeros((M, lda))
    B = np.zeros((K, ldb))
    operand = lambda r, c: (split_inputs(r, c, rng, 3.0) if r >= 4 and c >= 5 else
                            (rng.uniform(0, 1, (r, c)) - 0.5) * np.exp(3.0 * rng.standard_normal((r, c))))
    A[:, :K] = operand(M, K)
    B[:, :N] = operand(K, N)
    A[M // 2, :K] = 0.0  # an all-zero row
    B[:, N // 2] = 0.0   # an all-zero column
    A[:, K:] = 1e300     # beyond the extents: never read
    B[:, N:] = 1e300
    shift = 56 - 40
    bA, bB = dev.upload(A), dev.upload(B)
    dA, dB, fl = dev.alloc(4 * M), dev.alloc(4 * N), dev.alloc(8)
    dev.fill_u32(fl, 0, 2)
    dev.scale_pair(bA, M, K, lda, bB, N, ldb, ceil_mode, shift, dA, dB, fl)
    gA, gB = dev.download(dA, np.int32, M), dev.download(dB, np.int32, N)
    flags = dev.download(fl, np.uint32, 2)
    for x in (bA, bB, dA, dB, fl):
        x.free()
    dev.bufs.clear()
    wA, fA = oracle.scale(np.ascontiguousarray(A[:, :K]), M, K, 0, ceil_mode, shift)
    wB, fB = oracle.scale(np.ascontiguousarray(B[:, :N]), K, N, 1, ceil_mode, shift)
    np.testing.assert_array_equal(gA, wA)
    np.testing.assert_array_equal(gB, wB)
    assert list(flags) == [fA, fB] == [0, 0]


def test_scale_pair_flags(dev, oracle):
    """Range flags of the pair: Inf/NaN (4), a nonzero maximum below 2^-126 (2), above the largest BF16 (1),
    A's into flags[0] and B's into flags[1], as oz_scale_f64 reports them; the launch zeroes the other
    flag slot it is given (the next pass's), and ORs into its own without clearing it first."""
    M, N, K = 64, 48, 96
    A = np.ones((M, K))
    B = np.ones((K, N))
    A[3, 5] = np.inf
    A[7, :] = 2.0 ** -130
    B[:, 9] = 2.0 ** 129
    B[11, 2] = np.nan
    bA, bB = dev.upload(A), dev.upload(B)
    dA, dB, fl = dev.alloc(4 * M), dev.alloc(4 * N), dev.alloc(16)
    dev.fill_u32(fl, 0xFFFFFFFF, 4)
    dev.fill_u32(fl, 8, 1)  # a bit already set in this pass's slot (the launch ORs into it)
    dev.scale_pair(bA, M, K, K, bB, N, N, 1, 16, dA, dB, fl, fl.offset(8))
    both = dev.download(fl, np.uint32, 4)
    assert list(both[2:]) == [0, 0] and both[0] & 8 and both[1] == 0xFFFFFFFF
    dev.fill_u32(fl, 0, 2)
    dev.scale_pair(bA, M, K, K, bB, N, N, 1, 16, dA, dB, fl)
    flags = dev.download(fl, np.uint32, 2)
    gA, gB = dev.download(dA, np.int32, M), dev.download(dB, np.int32, N)
    for x in (bA, bB, dA, dB, fl):
        x.free()
    dev.bufs.clear()
    wA, fA = oracle.scale(A, M, K, 0, 1, 16)
    wB, fB = oracle.scale(B, K, N, 1, 1, 16)
    assert list(flags) == [fA, fB] == [4 | 2, 4 | 1]
    np.testing.assert_array_equal(gA, wA)
    np.testing.assert_array_equal(gB, wB)


@pytest.mark.parametrize("M,N,K,nd,b", [(300, 520, 700, 3, 56), (256, 256, 64, 4, 70), (17, 5, 33, 5, 90)])
def test_split_pair_equals_single_splits(dev, oracle, M, N, K, nd, b):
    """oz2_split_pair_int8 writes exactly the planes of oz2_split_int8 on A (layout 2) and B (layout 3),
    padding zeros included, and they equal the oracle's residues."""
    rng = np.random.default_rng(M * 7 + K)
    A = split_inputs(M, K, rng, 1.5)
    B = split_inputs(K, N, rng, 1.5)
    moduli = moduli_for(b, nd, 4096)
    md = moduli_desc(moduli, nd)
    S = len(moduli)
    shift = b - 20 * (nd - 1)
    wA, _ = oracle.scale(A, M, K, 0, 1, shift)
    wB, _ = oracle.scale(B, K, N, 1, 1, shift)
    Mg, Ng, Kg = -(-M // 16) * 16 + 16, -(-N // 16) * 16, -(-K // 64) * 64 + 64
    bA, bB, bdA, bdB = dev.upload(A), dev.upload(B), dev.upload(wA), dev.upload(wB)
    pA, pB = dev.alloc(S * Mg * Kg), dev.alloc(S * Ng * Kg)
    qA, qB = dev.alloc(S * Mg * Kg), dev.alloc(S * Ng * Kg)
    dev.fill_u32(pA, 0x5A5A5A5A, S * Mg * Kg // 4)
    dev.fill_u32(pB, 0x5A5A5A5A, S * Ng * Kg // 4)
    dev.split_pair_int8(bA, M, K, K, bdA, bB, N, N, bdB, md, pA, pB, Mg, Ng, Kg)
    dev.split_int8(bA, M, K, K, 0, bdA, md, qA, 2, Mg, Kg, Mg * Kg)
    dev.split_int8(bB, K, N, N, 1, bdB, md, qB, 3, Ng, Kg, Ng * Kg)
    got = [dev.download(x, np.int8, S * r * Kg) for x, r in ((pA, Mg), (pB, Ng), (qA, Mg), (qB, Ng))]
    for x in (bA, bB, bdA, bdB, pA, pB, qA, qB):
        x.free()
    dev.bufs.clear()
    np.testing.assert_array_equal(got[0], got[2])
    np.testing.assert_array_equal(got[1], got[3])
    want_A = oracle.residues(A, M, K, 0, wA, nd, moduli)
    want_B = oracle.residues(B, K, N, 1, wB, nd, moduli)
    pa = from_blocks(got[0].reshape(S, -1), Mg, Kg)
    pb = from_blocks(got[1].reshape(S, -1), Ng, Kg)
    np.testing.assert_array_equal(pa[:, :M, :K], want_A)
    np.testing.assert_array_equal(pb[:, :N, :K], want_B.transpose(0, 2, 1))
    assert not pa[:, M:, :].any() and not pa[:, :, K:].any() and not pb[:, N:, :].any() and not pb[:, :, K:].any()
