"""Pins the oracle's composition: orc_layer_forward and orc_model_forward.

The kernels the oracle composes are pinned one by one elsewhere
(test_oracle_kernels.py, test_oracle_pins.py). What those leave open is the
order they are wired in, so this file restates one decoder layer and the model
head in float64, written directly from the reference rather than from the
oracle:
- src/metal_encode.m:124-187 (encode_layer): norm -> q, k, v -> RoPE on q with
  the query factor and on k without -> rotated k and raw v appended to the cache
  at `length` -> scores/attend over positions [0, length+t] -> o -> residual
  x+o -> post norm of x+o -> gate, up -> SiLU(gate)*up -> down -> residual
  (x+o)+down;
- src/metal_encode.m:204-210: final norm and the tied head on the LAST row;
- src/metal_runtime.m:386-401: embedding rows widened, positions length+i;
- kernel formulas from src/metal_kernels.metal: norm :29-44, element :46-57,
  rope :59-78 (factor 1 + 0.1 ln(1 + floor(pos/16384))), scores :80-114 (scale
  0.08838834764831845, softmax over p <= prefix+t), attend :116-132, weight()
  :136-144 (E4M3FN decode times the per-tensor scale).
The cos/sin tables are the oracle's YaRN, which is pinned bitwise to the
reference's own src/metal_yarn.c: YaRN evaluates its angle in fp32 by
definition, and a float64 angle differs by up to ~1e-3 rad at 16K positions.

The bytes (FP8 codes drawn from the 254 finite codes, BF16 norms 1+N(0,0.02),
a BF16 N(0,1) embedding) come from the library's seeded generators. The
per-tensor scales are this test's own small powers of two, so that scores have
a standard deviation near 2 and the softmax stays soft: a composition slip then
moves the result by far more than rounding does. Both oracle schedules must agree with float64 to
1e-5 of each row's max-abs. Eight planted composition mistakes, compiled into
oracle variants with -DORC_PLANT=n, must each fail the same comparison.
"""

import numpy as np
import pytest

import oracle_lib
from oracle_lib import MIRROR, REF

H, Q, KV, I = 3072, 4096, 1024, 9216
VOCAB = 131072
SHAPES = {"q": (Q, H), "k": (KV, H), "v": (KV, H), "o": (H, Q), "gate": (I, H), "up": (I, H),
          "down": (H, I)}
SCALES = {"q": 2.0 ** -12, "k": 2.0 ** -12, "v": 2.0 ** -12, "o": 2.0 ** -11,
          "gate": 2.0 ** -12, "up": 2.0 ** -12, "down": 2.0 ** -13}
EPS = float(np.float32(1e-5))
SCORE_SCALE = 0.08838834764831845
TOL = 1e-5
PLANTS = oracle_lib.PLANTS


def e4m3_f64():
    """weight() of src/metal_kernels.metal:136-144 without the scale, in float64."""
    codes = np.arange(256)
    e = (codes >> 3) & 15
    f = (codes & 7).astype(np.float64)
    mag = np.where(e == 0, f * 2.0 ** -9, (1.0 + f / 8.0) * np.exp2(e.astype(np.float64) - 7))
    return np.where(codes & 128, -mag, mag)


def widen(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32).astype(np.float64)


class Weights:
    """A seeded model of `layers` layers in both forms: codes/bits for the
    oracle and decoded float64 for the restatement."""

    def __init__(self, seed, layers):
        import lunelette_amd.synthetic as syn
        table = e4m3_f64()
        self.layers = []
        for i in range(layers):
            L = syn.layer(seed, i)
            for name in SHAPES:
                assert L[name].shape == SHAPES[name]
                L["scale_" + name] = SCALES[name]
            self.layers.append(L)
        self.embedding = syn.normal_bf16(seed, 0, VOCAB * H, 0.0, 1.0).reshape(VOCAB, H)
        self.final_norm = syn.final_norm(seed)
        self.f64 = []
        for L in self.layers:
            d = {"gin": widen(L["input_norm"]), "gpost": widen(L["post_norm"])}
            for name in SHAPES:
                d[name] = table[L[name]] * L["scale_" + name]
            self.f64.append(d)


def rmsnorm(x, gamma):
    return gamma * (x / np.sqrt((x * x).sum(1, keepdims=True) / x.shape[1] + EPS))


def rope(x, cos, sin, factor=None):
    n = x.shape[0]
    xh = x.reshape(n, -1, 128)
    rot = np.concatenate([-xh[..., 64:], xh[..., :64]], axis=-1)
    out = xh * cos[:, None, :] + rot * sin[:, None, :]
    if factor is not None:
        out = out * factor[:, None, None]
    return out.reshape(n, -1)


def tables(length, count):
    cos = np.empty((count, 128))
    sin = np.empty((count, 128))
    for t in range(count):
        rc, c, s = oracle_lib.yarn(length + t)
        assert rc == 0
        cos[t], sin[t] = c, s
    pos = np.arange(length, length + count)
    factor = 1.0 + 0.1 * np.log(1.0 + np.floor(pos / 16384.0))
    return cos, sin, factor


def layer_f64(w, x, keys, values, length):
    """One decoder layer in float64; keys/values are position-major [C][1024]
    caches, appended in place (src/metal_encode.m:124-187)."""
    n = x.shape[0]
    cos, sin, factor = tables(length, n)
    xin = rmsnorm(x, w["gin"])
    q = xin @ w["q"].T
    k = xin @ w["k"].T
    v = xin @ w["v"].T
    rq = rope(q, cos, sin, factor)
    rk = rope(k, cos, sin)
    keys[length:length + n] = rk
    values[length:length + n] = v
    attn = np.empty((n, Q))
    for t in range(n):
        last = length + t
        for g in range(8):
            K = keys[:last + 1, g * 128:(g + 1) * 128]
            V = values[:last + 1, g * 128:(g + 1) * 128]
            s = (rq[t, g * 512:(g + 1) * 512].reshape(4, 128) @ K.T) * SCORE_SCALE
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            attn[t, g * 512:(g + 1) * 512] = (p @ V).reshape(-1)
    residual = x + attn @ w["o"].T
    post = rmsnorm(residual, w["gpost"])
    gate = post @ w["gate"].T
    up = post @ w["up"].T
    gated = gate / (1.0 + np.exp(-gate)) * up
    return residual + gated @ w["down"].T


def head_f64(weights, x_last):
    final = rmsnorm(x_last[None, :], widen(weights.final_norm))[0]
    logits = np.empty(VOCAB)
    for r in range(0, VOCAB, 16384):
        logits[r:r + 16384] = widen(weights.embedding[r:r + 16384]) @ final
    return logits


def rel_err(got, want):
    """max |got - want| over each row, divided by that row's max |want|."""
    got = np.atleast_2d(np.asarray(got, np.float64))
    want = np.atleast_2d(want)
    return float(np.max(np.abs(got - want).max(1) / np.abs(want).max(1)))


class Case:
    """A run of the oracle and of the float64 restatement over the same calls.

    calls: list of (length, ids). Positions below the first call's length are a
    seeded KV prefix written into both caches."""

    def __init__(self, weights, capacity, calls, prefix_seed=0):
        self.w = weights
        self.capacity = capacity
        self.calls = calls
        self.prefix = calls[0][0]
        rng = np.random.default_rng(prefix_seed)
        n_layers = len(weights.layers)
        self.prefix_kv = [(rng.standard_normal((self.prefix, KV), np.float32),
                           rng.standard_normal((self.prefix, KV), np.float32))
                          for _ in range(n_layers)]
        self.want = self._reference()

    def _reference(self):
        caches = []
        for K0, V0 in self.prefix_kv:
            keys = np.zeros((self.capacity, KV))
            values = np.zeros((self.capacity, KV))
            keys[:self.prefix] = K0
            values[:self.prefix] = V0
            caches.append((keys, values))
        out = []
        for length, ids in self.calls:
            x = widen(self.w.embedding[np.asarray(ids)])
            layers = []
            for i, f in enumerate(self.w.f64):
                x = layer_f64(f, x, caches[i][0], caches[i][1], length)
                layers.append(x.copy())
            out.append({"layers": layers, "logits": head_f64(self.w, x[-1]),
                        "kv": [(c[0][length:length + len(ids)].copy(),
                                c[1][length:length + len(ids)].copy()) for c in caches]})
        return out

    def errors(self, schedule, lib=None, layers=True):
        """Worst relative error over layer outputs (when `layers`), appended KV
        rows and logits."""
        model = oracle_lib.HostModel(self.w.embedding.reshape(-1), self.w.final_norm,
                                     self.w.layers, self.capacity, lib=lib)
        C = self.capacity
        for i, (K0, V0) in enumerate(self.prefix_kv):
            for cache, rows in ((model.keys, K0), (model.values, V0)):
                view = cache[i * 8 * C * 128:(i + 1) * 8 * C * 128].reshape(8, C, 128)
                view[:, :self.prefix, :] = rows.reshape(self.prefix, 8, 128).transpose(1, 0, 2)
        worst = {"layers": 0.0, "kv": 0.0, "logits": 0.0}
        for (length, ids), want in zip(self.calls, self.want):
            # Layer by layer from the same fp32 input the oracle received; the
            # oracle's layer output then continues the oracle's own chain.
            x = np.ascontiguousarray(
                widen(self.w.embedding[np.asarray(ids)]).astype(np.float32))
            for i in range(len(self.w.layers) if layers else 0):
                xin = x.astype(np.float64)
                model.layer_forward(schedule, i, x.reshape(-1), length, len(ids))
                snapshot = {
                    "keys": model.kv(i, 0, length, len(ids)),
                    "values": model.kv(i, 1, length, len(ids))}
                cache = self._restated_layer(i, xin, length)
                worst["layers"] = max(worst["layers"], rel_err(x, cache["x"]))
                worst["kv"] = max(worst["kv"], rel_err(snapshot["keys"], cache["keys"]),
                                  rel_err(snapshot["values"], cache["values"]))
            # The model forward overwrites the same KV rows with its own chain.
            logits = model.forward(schedule, ids, length)
            worst["logits"] = max(worst["logits"], rel_err(logits, want["logits"]))
            worst["kv"] = max(worst["kv"], *(
                max(rel_err(model.kv(i, 0, length, len(ids)), want["kv"][i][0]),
                    rel_err(model.kv(i, 1, length, len(ids)), want["kv"][i][1]))
                for i in range(len(self.w.layers))))
        return worst

    def _restated_layer(self, i, xin, length):
        """Float64 layer i from the oracle's fp32 input, over a cache holding
        the same prefix rows the restated chain wrote before `length`."""
        keys = np.zeros((self.capacity, KV))
        values = np.zeros((self.capacity, KV))
        keys[:self.prefix] = self.prefix_kv[i][0]
        values[:self.prefix] = self.prefix_kv[i][1]
        for (l, ids), want in zip(self.calls, self.want):
            if l >= length:
                break
            keys[l:l + len(ids)] = want["kv"][i][0]
            values[l:l + len(ids)] = want["kv"][i][1]
        x = layer_f64(self.w.f64[i], xin, keys, values, length)
        n = xin.shape[0]
        return {"x": x, "keys": keys[length:length + n], "values": values[length:length + n]}


@pytest.fixture(scope="module")
def weights():
    return Weights(20260101, 2)


@pytest.fixture(scope="module")
def case_start(weights):
    """Prefill of 5 ids at position 0, then a 1-id decode at position 5."""
    rng = np.random.default_rng(3)
    ids = rng.integers(0, VOCAB, 6)
    return Case(weights, 64, [(0, ids[:5]), (5, ids[5:])])


@pytest.fixture(scope="module")
def case_long(weights):
    """5 ids at positions 16382..16386 (the query factor turns 1+0.1 ln 2 at
    16384) over a seeded 16382-row prefix, then a 1-id decode at 16387."""
    rng = np.random.default_rng(4)
    ids = rng.integers(0, VOCAB, 6)
    return Case(weights, 16392, [(16382, ids[:5]), (16387, ids[5:])], prefix_seed=5)


def test_restatement_keeps_softmax_soft(weights, case_start):
    # The premise of the tolerance: scores of order 1, so no head is one-hot and
    # each composition term moves the output by far more than rounding.
    f = weights.f64[0]
    x = widen(weights.embedding[:5])
    xin = rmsnorm(x, f["gin"])
    q = xin @ f["q"].T
    k = xin @ f["k"].T
    s = (q[:, :128] @ k[:, :128].T) * SCORE_SCALE
    assert 0.5 < np.std(s) < 5.0


@pytest.mark.parametrize("schedule", [REF, MIRROR], ids=["ref", "mirror"])
@pytest.mark.parametrize("which", ["start", "long"])
def test_oracle_composition_matches_float64(schedule, which, case_start, case_long):
    case = case_start if which == "start" else case_long
    worst = case.errors(schedule)
    assert worst["layers"] <= TOL, worst
    assert worst["kv"] <= TOL, worst
    assert worst["logits"] <= TOL, worst


@pytest.fixture(scope="module")
def planted(tmp_path_factory):
    """Oracle builds with one planted composition mistake each."""
    return oracle_lib.build_planted(sorted(PLANTS), tmp_path_factory.mktemp("planted"))


@pytest.mark.parametrize("plant", sorted(PLANTS), ids=lambda n: PLANTS[n].replace(" ", "_"))
def test_planted_composition_mistake_fails(plant, planted, case_start, case_long):
    # Each mistake must miss the float64 restatement by at least 100x the
    # tolerance on one of the two cases (the query factor only differs from 1
    # at positions >= 16384, so plants 3 and 8 show on the long case alone).
    worst = 0.0
    for case in (case_start, case_long):
        worst = max(worst, *case.errors(MIRROR, lib=planted[plant], layers=False).values())
        if worst > 100 * TOL:
            break
    assert worst > 100 * TOL, (PLANTS[plant], worst)
