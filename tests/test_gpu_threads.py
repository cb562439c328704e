"""Calls from several host threads (reference context.cpp:19, :152 and README.md:81-85: one
process-wide lock serializes every Context's use of the device; arguments are validated before it).

Threads call the public API at the same time, on their own Contexts and on one shared Context, with
Scheme II INT8, Scheme II with the default Options (BFP8) and Scheme I BF16, and with resident
operands; every result must be the one the same call gives alone, bit for bit, and an invalid call
in one thread must fail there without disturbing the others. (ctypes releases the GIL for the
duration of each library call, so the calls overlap inside the library.)
"""
import threading

import numpy as np
import pytest

import oztt_amd as oz

pytestmark = pytest.mark.gpu

CASES = [
    ("II-INT8", oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8), 256, 192, 320, 1),
    ("II-default", oz.Options(), 200, 256, 128, 2),
    ("I-BF16", oz.Options(scheme=oz.Scheme.I, format=oz.Format.BF16, slices=6), 128, 256, 512, 3),
]


def inputs(case):
    _, _, m, n, k, seed = case
    return oz.eval_inputs(seed, 1.0, m * k, k * n)


@pytest.fixture(scope="module")
def expected():
    ctx = oz.Context()
    out = {}
    for case in CASES:
        name, o, m, n, k, _ = case
        a, b = inputs(case)
        out[name] = ctx.multiply(a, b, m, n, k, o)
    ctx.close()
    return out


def run_threads(targets):
    errors = []

    def wrap(fn):
        try:
            fn()
        except BaseException as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=wrap, args=(t,)) for t in targets]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=240)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    if errors:
        raise errors[0]


def bits(x):
    return np.ascontiguousarray(x).view(np.uint64)


@pytest.mark.parametrize("shared", [False, True], ids=["own-contexts", "shared-context"])
def test_concurrent_calls_give_the_sequential_results(expected, shared):
    common = oz.Context() if shared else None
    results = {}

    def worker(t):
        ctx = common if shared else oz.Context()
        try:
            for rep in range(3):
                case = CASES[(t + rep) % len(CASES)]
                name, o, m, n, k, _ = case
                a, b = inputs(case)
                results[(t, rep)] = (name, ctx.multiply(a, b, m, n, k, o))
        finally:
            if not shared:
                ctx.close()

    run_threads([lambda t=t: worker(t) for t in range(4)])
    assert len(results) == 12
    for name, c in results.values():
        np.testing.assert_array_equal(bits(c), bits(expected[name]))
    if common:
        common.close()


def test_invalid_call_fails_only_in_its_thread(expected):
    ctx = oz.Context()
    outcome = {}

    def bad():
        a = np.ones(64 * 64)
        a[5] = np.nan
        try:
            ctx.multiply(a, np.ones(64 * 64), 64, 64, 64, oz.Options(scheme=oz.Scheme.II, format=oz.Format.INT8))
            outcome["bad"] = "no error"
        except ValueError as e:
            outcome["bad"] = e

    def good():
        case = CASES[0]
        name, o, m, n, k, _ = case
        a, b = inputs(case)
        outcome["good"] = ctx.multiply(a, b, m, n, k, o)

    run_threads([bad, good, bad, good])
    assert isinstance(outcome["bad"], ValueError)
    np.testing.assert_array_equal(bits(outcome["good"]), bits(expected["II-INT8"]))
    ctx.close()


def test_resident_operands_from_threads(expected):
    """Each thread multiplies its own resident pair on a shared Context, repeatedly (the kept plan)."""
    ctx = oz.Context()
    results = []

    def worker(case):
        name, o, m, n, k, _ = case
        a, b = inputs(case)
        A, B = ctx.upload(a, m, k), ctx.upload(b, k, n)
        for _ in range(2):
            c = np.empty(m * n)
            ctx.gemm_resident(A, B, c, o)
            results.append((name, c))
        A.close()
        B.close()

    run_threads([lambda c=c: worker(c) for c in CASES])
    assert len(results) == 2 * len(CASES)
    for name, c in results:
        np.testing.assert_array_equal(bits(c), bits(expected[name]))
    ctx.close()
