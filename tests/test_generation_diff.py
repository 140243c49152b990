"""The generation loop against the reference's own C, and its allocation
failures.

Differential (src/generation.c:36-136, built from source into
oracle/_ref/libref.so): the same scripted logits callback drives
lunelette_generate_with_logits_capacity of liblunelette_hip.so and of the
reference over seeded scenarios: contexts 256 and 4352, prompts of length 1,
limit - 1 and limit and in between, budgets 0..256, an EOS id that becomes the
maximum at a chosen step, exact ties, a NaN or Inf logit at a chosen step, a
callback failure at a chosen step, and invalid requests (prompt ids, lengths,
budgets, EOS ids, limits, missing pointers). Return code, every field of the
result (all 256 token slots, count, stop reason), the untouched result on
failure, and the callback's trace (prefix length and a digest of the prefix
ids on every call) must be identical. Diagnostics are free text and are only
required to be present on failure.

Allocation failure (tests/test_generation_alloc.c): through the test library's
host allocation seam, the nth allocation of a call fails for every n up to the
first call that allocates nothing more: the call returns -1 with a
diagnostic, leaves the result untouched and frees everything it allocated.
"""
import ctypes
import hashlib

import numpy as np
import pytest

import lunelette_amd as lh

import oracle_lib

VOCAB = lh.VOCAB
POOL = 16


def declare(l):
    l.lunelette_generate_with_logits_capacity.restype = ctypes.c_int
    l.lunelette_generate_with_logits_capacity.argtypes = [
        lh.LOGITS_FN, ctypes.c_void_p, lh.c_int64_p, ctypes.c_size_t, ctypes.c_size_t,
        ctypes.POINTER(lh.GenerationConfig), ctypes.POINTER(lh.GenerationResult),
        ctypes.c_char_p, ctypes.c_size_t]
    return l


@pytest.fixture(scope="module")
def libraries(product):
    ref = oracle_lib.load_ref()
    if ref is None:
        pytest.skip("oracle/_ref/libref.so is not built (the reference checkout is absent)")
    return declare(product), declare(ref)


@pytest.fixture(scope="module")
def pool():
    rng = np.random.default_rng(5)
    return rng.standard_normal((POOL, VOCAB)).astype(np.float32)


class Script:
    """A deterministic logits callback. At prefix length n it writes pool row
    (n mod POOL), then makes `winner(n)` the maximum (with `ties` equal
    copies at higher and lower ids), and at the chosen steps writes a NaN or
    Inf, makes EOS the maximum, or fails."""

    def __init__(self, pool, prompt_len, seed, eos, eos_step=None, fail_step=None,
                 bad_step=None, bad_value=np.nan, ties=0):
        self.pool, self.prompt_len, self.seed = pool, prompt_len, seed
        self.eos, self.eos_step, self.fail_step = eos, eos_step, fail_step
        self.bad_step, self.bad_value, self.ties = bad_step, bad_value, ties
        self.trace = []
        self.fn = lh.LOGITS_FN(self.call)

    def winner(self, n):
        return int((n * 2654435761 + self.seed * 40503) % VOCAB)

    def call(self, context, ids, count, logits, error, capacity):
        step = count - self.prompt_len
        prefix = np.ctypeslib.as_array(ids, shape=(count,))
        self.trace.append((count, hashlib.sha1(prefix.tobytes()).hexdigest()[:16]))
        if step == self.fail_step:
            return -1
        out = np.ctypeslib.as_array(logits, shape=(VOCAB,))
        out[:] = self.pool[count % POOL]
        top = float(out.max()) + 1.0
        win = self.eos if step == self.eos_step else self.winner(count)
        out[win] = top
        for k in range(self.ties):
            out[(win + 7919 * (k + 1)) % VOCAB] = top
        if step == self.bad_step:
            out[(win * 31 + 5) % VOCAB] = self.bad_value
        return 0


def run(l, script, prompt, count, limit, budget, eos, with_result=True):
    config = lh.GenerationConfig(budget, eos)
    result = lh.GenerationResult()
    ctypes.memset(ctypes.byref(result), 0x55, ctypes.sizeof(result))
    err = ctypes.create_string_buffer(256)
    rc = l.lunelette_generate_with_logits_capacity(
        script.fn, None, prompt.ctypes.data_as(lh.c_int64_p) if prompt is not None else None,
        count, limit, ctypes.byref(config), ctypes.byref(result) if with_result else None,
        err, 256)
    return rc, bytes(result), err.value, list(script.trace)


def fields(raw):
    r = lh.GenerationResult.from_buffer_copy(raw)
    return list(r.tokens), r.count, r.stop


def compare(libraries, pool, prompt, count, limit, budget, eos, with_result=True, **kw):
    got = []
    for l in libraries:
        script = Script(pool, count, **kw, eos=eos)
        got.append(run(l, script, prompt, count, limit, budget, eos, with_result))
    (rc, raw, err, trace), (rc_r, raw_r, err_r, trace_r) = got
    assert rc == rc_r, (rc, rc_r, err, err_r)
    assert trace == trace_r
    if rc == 0:
        assert fields(raw) == fields(raw_r)
        assert err == b""
    else:
        assert raw == raw_r == bytes([0x55]) * len(raw)
        assert err
    return rc, fields(raw) if rc == 0 else None


def test_scenarios_match_reference(libraries, pool):
    rng = np.random.default_rng(2026)
    stops = set()
    for case in range(160):
        limit = int(rng.choice([256, 4352]))
        kind = case % 4
        count = [1, limit - 1, limit, int(rng.integers(1, limit + 1))][kind]
        budget = int(rng.choice([0, 1, 256, int(rng.integers(0, 257))]))
        prompt = rng.integers(0, VOCAB, size=count).astype(np.int64)
        eos = int(rng.choice([2, int(rng.integers(0, VOCAB))]))
        # A prompt id equal to EOS is not a stop.
        prompt[0] = eos if case % 5 == 0 else prompt[0]
        kw = dict(seed=case, ties=int(rng.integers(0, 3)))
        event = case % 6
        step = int(rng.integers(0, max(1, min(budget, limit - count) + 1)))
        if event == 1:
            kw["eos_step"] = step
        elif event == 2:
            kw["fail_step"] = step
        elif event == 3:
            kw["bad_step"], kw["bad_value"] = step, float(rng.choice([np.nan, np.inf, -np.inf]))
        elif event == 4:
            kw["eos_step"], kw["fail_step"] = step, step + 1
        rc, res = compare(libraries, pool, prompt, count, limit, budget, eos, **kw)
        if res is not None:
            stops.add(res[2])
    assert stops == {0, 1, 2}


def test_every_eos_step_matches_reference(libraries, pool):
    prompt = np.arange(5, dtype=np.int64)
    for step in range(0, 40):
        rc, res = compare(libraries, pool, prompt, 5, 256, 40, 17, seed=step, eos_step=step)
        assert rc == 0 and res[1] == step + 1 and res[2] == 1


def test_invalid_requests_match_reference(libraries, pool):
    ok = np.array([1, 2, 3], np.int64)
    for ids, count, limit, budget, eos in (
            (ok, 0, 256, 4, 2), (ok, 3, 255, 4, 2), (ok, 3, 4353, 4, 2), (ok, 3, 17920, 4, 2),
            (ok, 3, 256, 257, 2), (ok, 3, 256, 4, -1), (ok, 3, 256, 4, VOCAB),
            (np.array([1, -1, 3], np.int64), 3, 256, 0, 2),
            (np.array([1, 2, VOCAB], np.int64), 3, 4352, 4, 2),
            (np.zeros(257, np.int64), 257, 256, 4, 2), (None, 3, 256, 4, 2)):
        compare(libraries, pool, ids, count, limit, budget, eos, seed=1)
    compare(libraries, pool, ok, 3, 256, 4, 2, with_result=False, seed=1)


@pytest.fixture(scope="module")
def seams():
    l = declare(lh.test_lib())
    yield l
    l.lunelette_metal_test_fail_host_allocation(0)


@pytest.mark.parametrize("limit", [256, 4352])
def test_allocation_failures_clean_up(seams, pool, limit):
    prompt = np.array([1], np.int64)
    base = seams.lunelette_metal_test_live_host_allocations()
    nth = 1
    while True:
        seams.lunelette_metal_test_fail_host_allocation(nth)
        script = Script(pool, 1, seed=3, eos=2, fail_step=0)
        rc, raw, err, trace = run(seams, script, prompt, 1, limit, 32, 2)
        assert rc == -1 and raw == bytes([0x55]) * len(raw) and err
        assert seams.lunelette_metal_test_live_host_allocations() == base
        if trace:
            break   # every allocation before the first callback succeeded
        assert b"allocation" in err
        nth += 1
    assert nth == 3   # the prefix and the logits scratch
    seams.lunelette_metal_test_fail_host_allocation(0)
    rc, raw, _, _ = run(seams, Script(pool, 1, seed=3, eos=2), prompt, 1, limit, 32, 2)
    assert rc == 0 and fields(raw)[1] == 32
    assert seams.lunelette_metal_test_live_host_allocations() == base
