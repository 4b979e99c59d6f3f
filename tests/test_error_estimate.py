"""The prefill MFMA kernel's per-row rounding-error estimate (kernels/attn_prefill.hip, kEstZ / kEstBudget, the `est` /
residual expressions of attn_prefill_kernel and prefill_split_merge, and the staging's stochastic rounding f16_sr /
sr_bits), checked on the CPU against an emulation of the kernel's rounding: the scaled query y = Q * log2(e) / sqrt(d)
(fp32) enters the scores as two fp16 parts hi = fp16(y), lo = fp16(y - hi); K and V are staged to fp16 with the
kernel's stochastic rounding (its hash and bit manipulation restated here exactly, so the emulation rounds each element
as the GPU does); the softmax weights P are rounded to nearest; sums in high precision; all against the exact fp64
softmax. Rows whose estimate passes (1.5 sqrt(var) + ln2 |r| sqrt(K) (V + O) <= 1e-3, r = y - hi - lo) are the rows
the kernel keeps; every other row tile is recomputed with split operands.

The cases span the windows the MFMA route takes (65 keys and up: rows below position 128 run in fp32), score scales
0.5 to 30, the outlier shapes the estimate's bounds must cover, q, K and V projected from shared low-rank hidden
states (K and V correlate, as in a transformer, and a rounding of the query, common to every key of the row, would add
up coherently: the reason the kernel splits the query), and value rows that repeat - in runs, alternating, or at
scattered positions like a token recurring in a prompt - where rounding to nearest gives equal rows equal errors that
add up coherently: the reason the staging rounds stochastically. Reference semantics: ref_ops.cpp:188-214 computes
the row in fp32 for any input; tests/test_ops.cpp:196-216 holds its SIMD tier to the scalar one for any data."""
import importlib.util
import os

import numpy as np
import pytest

U = 2.0 ** -11          # kEstU: fp16 unit roundoff
LN2 = float(np.log(2.0))
Z, BUDGET = 1.5, 1e-3   # kEstZ, kEstBudget
TILE = 64               # keys per tile (kBN): the tile statistics are per-tile maxima
ROWS_PER_TILE = 128     # packed query rows of one MFMA row tile (kRowsPerBlock): flagged or kept together
M32 = np.uint64(0xFFFFFFFF)


def f16(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def sr_bits(rows, g, hd):
    """[len(rows), hd] words of sr_bits(row, g, d, hd) (attn_prefill.hip): lowbias32 of row * 0x9E3779B1 +
    (g * hd + d) * 0x85EBCA77 + 0x27D4EB2F, in 32-bit arithmetic."""
    r = np.asarray(rows, np.uint64)[:, None] & M32
    d = np.arange(hd, dtype=np.uint64)[None, :]
    x = (r * np.uint64(0x9E3779B1) + (np.uint64(g * hd) + d) * np.uint64(0x85EBCA77) + np.uint64(0x27D4EB2F)) & M32
    x ^= x >> np.uint64(16)
    x = (x * np.uint64(0x7FEB352D)) & M32
    x ^= x >> np.uint64(15)
    x = (x * np.uint64(0x846CA68B)) & M32
    x ^= x >> np.uint64(16)
    return x.astype(np.uint32)


def f16_sr(x, r13):
    """f16_sr (attn_prefill.hip) on float32 x with 13 random bits r13: (bits(x) + r13) with the low 13 bits cleared,
    for magnitudes in [2^-14, 2^15); rounding to nearest elsewhere. Returned as float64."""
    x32 = np.asarray(x, np.float32)
    b = x32.view(np.uint32)
    mag = b & np.uint32(0x7FFFFFFF)
    t = ((b + np.asarray(r13, np.uint32)) & np.uint32(0xFFFFE000)).view(np.float32)
    ok = (mag >= np.uint32(0x38800000)) & (mag < np.uint32(0x47000000))
    return np.where(ok, t, x32).astype(np.float16).astype(np.float64)


def stage(k, v, g=0, row0=0):
    """K and V rows row0, row0 + 1, ... of KV head g as the staging writes them: one hash word per element, bits
    0..12 for K and 13..25 for V."""
    bits = sr_bits(np.arange(row0, row0 + len(k)), g, k.shape[1])
    return f16_sr(k, bits & np.uint32(0x1FFF)), f16_sr(v, (bits >> np.uint32(13)) & np.uint32(0x1FFF))


def make(kind, n, hd, qscale, rng):
    q = rng.standard_normal(hd) * qscale
    k = rng.standard_normal((n, hd))
    v = rng.standard_normal((n, hd))
    if kind == "kout":      # 1 % of the key rows x 8
        k[rng.choice(n, max(1, n // 100), replace=False)] *= 8
    elif kind == "vout":    # 1 % of the value rows x 8
        v[rng.choice(n, max(1, n // 100), replace=False)] *= 8
    elif kind == "align":   # the query along one key
        j = rng.integers(n)
        q = k[j] / np.linalg.norm(k[j]) * np.linalg.norm(q)
    elif kind == "lowrank":  # keys and query in a 4-dimensional subspace
        b = rng.standard_normal((4, hd))
        k = rng.standard_normal((n, 4)) @ b / 2 + 0.1 * k
        q = (rng.standard_normal(4) @ b / 2) * qscale
    elif kind == "kmean":   # a large component common to every key
        mu = rng.standard_normal(hd)
        k = k + mu * (5 / np.linalg.norm(mu))
    elif kind == "vmean":   # a large component common to every value
        v = v + 3.0
    return q, k, v


def hidden(rng, n, hd, rank):
    """n hidden states of width 4 hd on a rank-`rank` subspace plus 10 % noise, and the key projection."""
    dm = 4 * hd
    a = rng.standard_normal((n, rank))
    b = rng.standard_normal((rank, dm))
    wk = rng.standard_normal((dm, hd)) / np.sqrt(dm)
    return a, b, wk, dm


def correlated(rng, n, hd, rank, vmix, qscale, qproj):
    """q, K = h Wk and V = h (vmix Wk + (1 - vmix) R) from shared low-rank hidden states h; q either random or the
    projection of one of the same hidden states (a query that attends to its own context)."""
    a, b, wk, dm = hidden(rng, n, hd, rank)
    wv = vmix * wk + (1 - vmix) * rng.standard_normal((dm, hd)) / np.sqrt(dm)
    h = a @ b / np.sqrt(rank) + 0.1 * rng.standard_normal((n, dm))
    if qproj:
        q = (h[rng.integers(n)] @ (rng.standard_normal((dm, hd)) / np.sqrt(dm))) * qscale
    else:
        q = rng.standard_normal(hd) * qscale
    return q, h @ wk, h @ wv


def scaled_query(q):
    hd = q.size
    return (q.astype(np.float32) * np.float32(np.log2(np.e) / np.sqrt(hd))).astype(np.float64)


def query_parts(qh):
    """(hi + lo, r): the query the MFMAs multiply and its residual (both differences exact, as in the kernel)."""
    hi = f16(qh)
    lo = f16(qh - hi)
    return hi + lo, qh - hi - lo


def emulate(q, k, v, split_q=True, sr=True, g=0):
    """(max-abs error of the fp16-operand row against fp64, the kernel's inputs to the estimate), keys at positions
    0, 1, ... of KV head g. split_q=False is the query rounded once and sr=False K and V rounded to nearest (the
    kernel before the split and before the stochastic staging), kept for the planted-mistake checks."""
    qh = scaled_query(q)
    s_ex = qh @ k.T
    w = np.exp2(s_ex - s_ex.max())
    ref = (w @ v) / w.sum()
    qq = query_parts(qh)[0] if split_q else f16(qh)
    kk, vv = stage(k, v, g) if sr else (f16(k), f16(v))
    s = qq @ kk.T
    p = f16(np.exp2(s - s.max()))
    l = p.sum()
    o = (p @ vv) / l
    return float(np.abs(o - ref).max()), qh, p, l, o


def estimate(qh, k, v, p, l, o, drop_v_term=False, u=U, sr=True, query_rounded=False):
    """(sqrt(var), residual bound) as the kernel evaluates them: var = (sum p^2 / l^2) [2 ln2^2 (c u^2/3) (|y|^2/d) K
    (V^2 + O^2) + (u^2/3)(c V^2 + 2 (V^2 + O^2))], c = 3 for stochastically rounded K and V (variance up to u^2 x^2)
    and 1 for rounding to nearest (u^2 x^2 / 3), plus 1 in the score term when the query is rounded once; K the
    largest per-tile max of |k_j|^2, V the largest |v| element, O the row's largest output; the residual bound
    ln2 |r| sqrt(K) (V + O)."""
    hd = qh.size
    nt = (len(k) + TILE - 1) // TILE
    kmx = max(float(np.max(np.sum(k[t * TILE:(t + 1) * TILE] ** 2, 1))) for t in range(nt))
    vmx = float(np.abs(v).max())
    om = float(np.abs(o).max())
    om2, vg2 = om * om, vmx * vmx
    qn2 = float(qh @ qh) / hd
    c = 3.0 if sr else 1.0
    c1 = 2 * LN2 * LN2 * ((c + (1.0 if query_rounded else 0.0)) * u * u / 3)
    c2 = 0.0 if drop_v_term else u * u / 3
    var = float(np.sum(p * p)) / (l * l) * (c1 * qn2 * kmx * (vg2 + om2) + c2 * (c * vg2 + 2 * (vg2 + om2)))
    r = query_parts(qh)[1]
    coh = LN2 * float(np.linalg.norm(r)) * np.sqrt(kmx) * (vmx + om)
    return float(np.sqrt(var)), coh


def kept(est):
    sv, coh = est
    return Z * sv + coh <= BUDGET


FLAT_TOL = 1.0 / 4096   # kFlatTol


def flat_row(p):
    """The kernel's flatness test (kFlatTol): keys * sum p^2 <= (sum p)^2 (1 + tol), equality when every weight is
    equal. Such a row is recomputed whatever its estimate."""
    return len(p) * float(np.sum(p * p)) <= float(np.sum(p)) ** 2 * (1 + FLAT_TOL)


# ------------------------------------------------------------------------------------------ stochastic rounding

def test_stochastic_rounding_lands_on_a_neighbour_and_is_unbiased():
    """f16_sr returns one of x's two fp16 neighbours (x itself when representable), rounds to nearest outside
    [2^-14, 2^15), and rounds up with probability equal to x's fractional position between the neighbours: over
    65536 positions a value 0.3 ulp above an fp16 number rounds up 30 % of the time (+- 1 %), so the mean error is
    ~0 where rounding to nearest errs by -0.3 ulp every time."""
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(20000) * np.exp(rng.uniform(-8, 8, 20000))).astype(np.float32)
    r = rng.integers(0, 1 << 13, x.size).astype(np.uint32)
    y = f16_sr(x, r)
    lo = x.astype(np.float16)
    lo = np.where(lo.astype(np.float32) > x, np.nextafter(lo, np.float16(-np.inf)), lo).astype(np.float64)
    hi = np.nextafter(lo.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    inside = (np.abs(x) >= 2.0 ** -14) & (np.abs(x) < 2.0 ** 15)
    assert np.all((y[inside] == lo[inside]) | (y[inside] == hi[inside]))
    assert np.array_equal(y[~inside], f16(x[~inside]))
    exact = np.float16(rng.standard_normal(1000)).astype(np.float32)
    assert np.array_equal(f16_sr(exact, rng.integers(0, 1 << 13, 1000).astype(np.uint32)), exact.astype(np.float64))
    base = np.float32(4.0 + 17 / 256)
    x03 = np.float32(base + 0.3 / 256)
    k, v = stage(np.full((65536, 1), x03), np.full((65536, 1), x03))
    for z in (k, v):
        up = float(np.mean(z > x03))
        assert abs(up - 0.3) < 0.01, up
    assert abs(float(np.mean(v - x03))) < 3e-5 and abs(float(f16(x03) - x03) + 0.3 / 256) < 1e-6


def test_stochastic_rounding_bits_are_independent_across_neighbours():
    """The hash words of neighbouring positions and dimensions look independent: the K and V bit fields of a 4096 x
    64 block are uniform (each of 8 bins within 3 % of its share) and uncorrelated between adjacent rows, adjacent
    dimensions and the K and V fields of one element (|corr| < 0.02)."""
    bits = sr_bits(np.arange(4096), 3, 64)
    kb = (bits & np.uint32(0x1FFF)).astype(np.float64)
    vb = ((bits >> np.uint32(13)) & np.uint32(0x1FFF)).astype(np.float64)
    for f in (kb, vb):
        counts = np.bincount((f.ravel() // 1024).astype(int), minlength=8)
        assert np.all(np.abs(counts / f.size - 0.125) < 0.03 * 0.125 * 8), counts
    for a, b in ((kb[1:], kb[:-1]), (kb[:, 1:], kb[:, :-1]), (kb, vb), (vb[1:], vb[:-1])):
        assert abs(np.corrcoef(a.ravel(), b.ravel())[0, 1]) < 0.02


# ------------------------------------------------------------------------------------------ families

KINDS = ["n01", "kout", "vout", "align", "lowrank", "kmean", "vmean"]
SCALES = [0.5, 1.0, 2.0, 5.0, 30.0]
WINDOWS = [65, 129, 256, 600, 2048]


def rows(seed):
    rng = np.random.default_rng(seed)
    for kind in KINDS:
        for qs in SCALES:
            for n in WINDOWS:
                for hd in (64, 128):
                    q, k, v = make(kind, n, hd, qs, rng)
                    yield (kind, qs, n, hd, q, k, v)


def corr_rows(seed):
    rng = np.random.default_rng(seed)
    for rank in (1, 2, 4, 8):
        for vmix in (0.5, 0.8, 1.0):
            for qs in (0.5, 1.0, 3.0):
                for n in (1024, 4096):
                    for hd in (64, 128):
                        for qproj in (False, True):
                            q, k, v = correlated(rng, n, hd, rank, vmix, qs, qproj)
                            yield (f"corr{rank}/{vmix}/{'qp' if qproj else 'qr'}", qs, n, hd, q, k, v)


def big_row(rng, hd, count=6):
    """A value row whose `count` largest elements are 4 + (m + f) 2^-8 for f in {0.49, 0.3, 0.1}: fp16 rounding to
    nearest errs by -f ulp (up to 1.9e-3) on each, the same for every copy of the row."""
    r = rng.standard_normal(hd)
    idx = rng.choice(hd, count, replace=False)
    r[idx] = rng.choice([-1, 1], count) * (4 + (rng.integers(0, 256, count) + rng.choice([0.49, 0.3, 0.1], count))
                                            / 256)
    return r


def repeated_rows(seed, count):
    """Rows whose value rows repeat (V carries no rotation, so a token repeated in the prompt repeats its value row):
    runs of L equal rows at a random place in the window (the query attending evenly or to the run, whose keys are
    aligned with it), two rows alternating over the whole window, or one row recurring at scattered positions every
    2-33 keys (its keys equal, aligned with the query, or unrelated)."""
    rng = np.random.default_rng(seed)
    for i in range(count):
        hd = (64, 128)[i % 2]
        n = int(rng.choice([129, 300, 600, 1000, 2048, 4096]))
        q = rng.standard_normal(hd) * float(rng.choice([0.5, 1.0, 2.0, 3.0]))
        k = rng.standard_normal((n, hd))
        v = rng.standard_normal((n, hd))
        kind = rng.choice(["run", "run-attended", "alternating", "scattered"])
        if kind == "alternating":
            v[0::2], v[1::2] = big_row(rng, hd), big_row(rng, hd)
            name = kind
        elif kind == "scattered":
            period = int(rng.choice([2, 3, 5, 7, 10, 16, 33]))
            pos = np.arange(int(rng.integers(0, period)), n, period)
            v[pos] = big_row(rng, hd)
            keys = rng.choice(["equal", "aligned", "unrelated"])
            along = q / np.linalg.norm(q) * np.sqrt(hd) * float(rng.choice([0.5, 1.0, 1.5]))
            if keys == "equal":
                k[pos] = along
            elif keys == "aligned":
                k[pos] += along
            name = f"scattered-{keys}/p{period}"
        else:
            L = int(rng.choice([1, 2, 4, 8, 16, 32, 64, n]))
            s0 = int(rng.integers(0, max(1, n - L)))
            v[s0:s0 + L] = big_row(rng, hd)
            if kind == "run-attended":
                m = min(L, n - s0)
                k[s0:s0 + m] = (q / np.linalg.norm(q) * np.linalg.norm(k[s0]) * 1.5
                                + 0.05 * rng.standard_normal((m, hd)))
            name = f"{kind}/L{L}"
        yield (name, 1.0, n, hd, q, k, v)


def with_emulation(cases, split_q=True, sr=True):
    return [c + emulate(*c[4:], split_q=split_q, sr=sr) for c in cases]


@pytest.fixture(scope="module")
def plain_cases():
    return [r for seed in (1, 2) for r in rows(seed)]


@pytest.fixture(scope="module")
def corr_cases():
    return list(corr_rows(3))


@pytest.fixture(scope="module")
def cases(plain_cases, corr_cases):
    return with_emulation(plain_cases + corr_cases)


@pytest.fixture(scope="module")
def repeated_cases():
    return list(repeated_rows(17, 400))


# ------------------------------------------------------------------------------------------ the estimate

def test_estimate_bounds_the_emulated_error(cases):
    """The emulated error stays below the estimate's sqrt(var) alone (measured: at most ~0.62 on these cases), so a
    row the kernel keeps errs by well under the 1e-3 bar; this holds on the correlated families too."""
    worst, at = 0.0, None
    for kind, qs, n, hd, q, k, v, err, qh, p, l, o in cases:
        sv, coh = estimate(qh, k, v, p, l, o)
        if err / sv > worst:
            worst, at = err / sv, (kind, qs, n, hd)
    assert worst < 0.95, f"emulated error up to {worst:.3f} sqrt(var) at {at}"


def test_residual_term_is_small(cases):
    """The query residual's outright bound stays a small part of the budget on every row the kernel could keep on
    the strength of the variance term alone (hi + lo leave ~2^-22 |y|; measured at most 1.4e-4)."""
    worst = 0.0
    for kind, qs, n, hd, q, k, v, err, qh, p, l, o in cases:
        sv, coh = estimate(qh, k, v, p, l, o)
        if Z * sv <= BUDGET:
            worst = max(worst, coh)
    assert worst < 0.2 * BUDGET, worst


def test_accepted_rows_meet_the_bar(cases):
    """Every row the estimate accepts is within 6e-4 of the exact result; the rows it rejects include the ones that
    miss 1e-3 (large scores)."""
    accepted = rejected = 0
    worst_acc = 0.0
    missed = []
    for kind, qs, n, hd, q, k, v, err, qh, p, l, o in cases:
        if kept(estimate(qh, k, v, p, l, o)):
            accepted += 1
            worst_acc = max(worst_acc, err)
        else:
            rejected += 1
        if err > BUDGET:
            missed.append((kind, qs, n, hd, err))
    assert accepted > 0 and rejected > 0
    assert worst_acc <= 6e-4, worst_acc
    assert missed, "no case misses the bar in fp16: the test would not exercise the rejection"


def reproducer():
    """Correlated K and V at rank 2 (V = h (0.8 Wk + 0.2 R)), 4096 keys, head_dim 64, q ~ 2 N(0,1): the row the
    estimate of an unsplit query keeps although it misses the bar."""
    n, hd, rank = 4096, 64, 2
    rng = np.random.default_rng(2023)
    a, b, wk, dm = hidden(rng, n, hd, rank)
    wv = 0.8 * wk + 0.2 * rng.standard_normal((dm, hd)) / np.sqrt(dm)
    h = a @ b / np.sqrt(rank) + 0.1 * rng.standard_normal((n, dm))
    q = rng.standard_normal(hd) * 2
    return q, h @ wk, h @ wv


def test_reproducer_row_is_flagged_or_within_the_bar():
    """With the query rounded once (and K, V rounded to nearest: that kernel), the row is kept and errs by 1.13e-3 -
    the query's rounding is shared by all 4096 keys and K, V correlate. With the split query and the stochastic
    staging it is within the bar and inside its estimate."""
    q, k, v = reproducer()
    err0, qh, p, l, o = emulate(q, k, v, split_q=False, sr=False)
    assert kept(estimate(qh, k, v, p, l, o, sr=False, query_rounded=True)) and err0 > BUDGET, err0
    err, qh, p, l, o = emulate(q, k, v)
    sv, coh = estimate(qh, k, v, p, l, o)
    assert err <= BUDGET and err <= 0.95 * sv, (err, sv)


def test_an_unsplit_query_underestimates_on_correlated_rows(corr_cases):
    """Planted mistake: the query rounded to fp16 once (the estimate then counting its rounding in the score term)
    is outgrown by the emulated error on correlated rows - the bound checked above would fail."""
    worst = 0.0
    for kind, qs, n, hd, q, k, v in corr_cases[::3]:
        err, qh, p, l, o = emulate(q, k, v, split_q=False, sr=False)
        worst = max(worst, err / estimate(qh, k, v, p, l, o, sr=False, query_rounded=True)[0])
    assert worst > 1.5, worst


def test_a_dropped_value_rounding_term_underestimates(cases):
    """Planted mistake: without the value- and weight-rounding term (u^2/3)(c V^2 + 2 (V^2 + O^2)) the estimate
    falls below the emulated error somewhere (short windows, small scores), so the check above would catch it."""
    worst = max(err / max(estimate(qh, k, v, p, l, o, drop_v_term=True)[0], 1e-30)
                for kind, qs, n, hd, q, k, v, err, qh, p, l, o in cases)
    assert worst > 1.0, worst


def test_a_halved_unit_roundoff_underestimates(cases):
    """Planted mistake: u = 2^-12 (half fp16's unit roundoff) halves the estimate, and the emulated error then exceeds
    it on some row."""
    worst = max(err / estimate(qh, k, v, p, l, o, u=U / 2)[0] for kind, qs, n, hd, q, k, v, err, qh, p, l, o in cases)
    assert worst > 1.1, worst


def tile_rows(rng, hd, rank, vmix, qscale, pos0, group=4):
    """One MFMA row tile as the kernel packs it: 128 / group consecutive query positions from pos0, each with its
    group heads (per-head query weights), q, K and V all projected from the same low-rank hidden states; row t sees
    keys [0, pos0 + t]."""
    n_pos = ROWS_PER_TILE // group
    n = pos0 + n_pos
    a, b, wk, dm = hidden(rng, n, hd, rank)
    wv = vmix * wk + (1 - vmix) * rng.standard_normal((dm, hd)) / np.sqrt(dm)
    h = a @ b / np.sqrt(rank) + 0.1 * rng.standard_normal((n, dm))
    k, v = h @ wk, h @ wv
    wq = rng.standard_normal((group, dm, hd)) / np.sqrt(dm) * qscale
    return [(h[pos0 + t] @ wq[j], k[:pos0 + t + 1], v[:pos0 + t + 1]) for t in range(n_pos) for j in range(group)]


def tiles(seed, count):
    rng = np.random.default_rng(seed)
    for i in range(count):
        hd = (64, 128)[i % 2]
        rank = (1, 2, 4, 8)[(i // 2) % 4]
        vmix = (0.6, 0.8, 1.0)[(i // 8) % 3]
        qscale = (0.5, 1.0, 2.0)[(i // 24) % 3]
        pos0 = int(rng.integers(256, 4096))
        yield (hd, rank, vmix, qscale, pos0), tile_rows(rng, hd, rank, vmix, qscale, pos0)


def judge_tile(rows_):
    """(tile kept, worst row error, worst err / sqrt(var)) with the kernel's rule: one row over budget flags all."""
    keep, worst, ratio = True, 0.0, 0.0
    for q, k, v in rows_:
        err, qh, p, l, o = emulate(q, k, v)
        est = estimate(qh, k, v, p, l, o)
        keep = keep and kept(est)
        worst = max(worst, err)
        ratio = max(ratio, err / est[0])
    return keep, worst, ratio


def test_row_tiles_from_shared_hidden_states():
    """Whole 128-row tiles (32 positions x 4 GQA heads, the query also projected from the hidden states): no row of
    a kept tile errs by more than 6e-4, every row stays within 0.95 sqrt(var), and some tiles are kept."""
    kept_tiles = 0
    for cfg, rows_ in tiles(11, 48):
        keep, worst, ratio = judge_tile(rows_)
        assert ratio < 0.95, (cfg, ratio)
        if keep:
            kept_tiles += 1
            assert worst <= 6e-4, (cfg, worst)
    assert kept_tiles > 0


# ------------------------------------------------------------------------------------------ repeated value rows

def test_repeated_value_rows_stay_within_the_bar(repeated_cases):
    """Value rows repeated in runs, alternating or at scattered positions, with elements 0.1-0.49 fp16 ulp off the
    grid: stochastically rounded, equal rows carry independent errors and the variance model holds - every row errs
    by less than 1.45 sqrt(var) (the largest elements, near the top of their rounding variance, make the estimate
    tight: measured up to ~1.3), so a kept row (1.5 sqrt(var) <= 1e-3) meets the bar; kept rows measured up to
    ~7e-4, and many rows are kept."""
    worst, at, worst_kept, n_kept = 0.0, None, 0.0, 0
    for kind, qs, n, hd, q, k, v in repeated_cases:
        err, qh, p, l, o = emulate(q, k, v)
        sv, coh = estimate(qh, k, v, p, l, o)
        if err / sv > worst:
            worst, at = err / sv, (kind, n, hd)
        if Z * sv + coh <= BUDGET:
            n_kept += 1
            worst_kept = max(worst_kept, err)
    assert worst < 0.95 * Z, f"emulated error up to {worst:.3f} sqrt(var) at {at}"
    assert worst_kept <= 8e-4, worst_kept
    assert n_kept > len(repeated_cases) // 4


def test_rounding_to_nearest_misses_the_bar_on_repeated_rows(repeated_cases):
    """Planted mistake: K and V rounded to nearest (with the estimate's constants for that rounding) - equal rows
    then round alike and their errors add up: the estimate keeps rows that miss the 1e-3 bar (measured: over a
    third of the scattered ones, at up to 1.97e-3)."""
    missed = 0
    for kind, qs, n, hd, q, k, v in repeated_cases[::2]:
        err, qh, p, l, o = emulate(q, k, v, sr=False)
        if kept(estimate(qh, k, v, p, l, o, sr=False)) and err > BUDGET:
            missed += 1
    assert missed >= 10, missed


def load_make_golden():
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "make_golden.py")
    spec = importlib.util.spec_from_file_location("make_golden", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_repeated_value_golden_cases():
    """The repeated-value golden cases (tests/golden/make_golden.py, REPEAT_CASES) on sampled rows - first, middle
    and last row of the call, heads spread over the KV groups, keys at their absolute positions and KV head, so the
    emulation stages each element with the kernel's own random bits: with rounding to nearest every sampled row errs
    by more than the bar while its estimate keeps it; with the stochastic staging every sampled row is within the
    bar. On the all-equal cases (`repeat_const_*`) the estimate keeps every sampled row and the error stays within
    4e-4 (every row of `repeat_const_chunk` is kept, so the GPU test sees the MFMA route's own result there)."""
    mg = load_make_golden()
    for i, case in enumerate(mg.REPEAT_CASES):
        name, n, pos0, H, KV, D = case[:6]
        q, k, v = mg.repeat_inputs(i, *case[1:])
        g = H // KV
        for r in (0, n // 2, n - 1):
            for h in range(0, H, max(g, H // 4)):
                ctx = pos0 + r + 1
                qq = q[r, h].astype(np.float64)
                kk, vv = k[:ctx, h // g].astype(np.float64), v[:ctx, h // g].astype(np.float64)
                err0, qh, p, l, o = emulate(qq, kk, vv, sr=False)
                assert err0 > BUDGET and kept(estimate(qh, kk, vv, p, l, o, sr=False)), (name, r, h, err0)
                err, qh, p, l, o = emulate(qq, kk, vv, g=h // g)
                assert err <= BUDGET, (name, r, h, err)
                if name.startswith("repeat_const"):
                    assert kept(estimate(qh, kk, vv, p, l, o)) and err <= 4e-4, (name, r, h, err)


def outlier_channel_rows(seed, count):
    """Keys with 1-4 channels shared by every key at magnitude 5-40 (+-20 %), which the query also weights (LLM keys
    carry such channels): the score term's |y|^2/d |k|^2 reading of sum_d y_d^2 k_d^2 assumes no such alignment."""
    rng = np.random.default_rng(seed)
    for i in range(count):
        hd = (64, 128)[i % 2]
        n = int(rng.choice([129, 300, 1000, 2048]))
        nd = int(rng.choice([1, 2, 4]))
        mag = float(rng.choice([5, 10, 20, 40]))
        qs = float(rng.choice([0.5, 1.0, 2.0]))
        dims = rng.choice(hd, nd, replace=False)
        k = rng.standard_normal((n, hd))
        v = rng.standard_normal((n, hd))
        q = rng.standard_normal(hd) * qs
        k[:, dims] = mag * (1 + 0.2 * rng.standard_normal((n, nd)))
        q[dims] = mag / 8 * rng.choice([-1, 1], nd) * qs
        yield mag, q, k, v


def test_shared_outlier_channels():
    """Keys with outlier channels the query weights: up to magnitude 10 the emulated error stays within 0.95 sqrt(var)
    (measured ~0.63); beyond, the estimate underestimates the score term (measured up to 1.15 sqrt(var) at 20 and
    2.0 at 40), but those keys also raise the largest key norm K, so the rows it keeps stay within 6e-4."""
    worst_small, worst_kept, n_kept = 0.0, 0.0, 0
    for mag, q, k, v in outlier_channel_rows(6, 240):
        err, qh, p, l, o = emulate(q, k, v)
        sv, coh = estimate(qh, k, v, p, l, o)
        if mag <= 10:
            worst_small = max(worst_small, err / sv)
        if kept((sv, coh)):
            n_kept += 1
            worst_kept = max(worst_kept, err)
    assert worst_small < 0.95, worst_small
    assert worst_kept <= 6e-4, worst_kept
    assert n_kept > 0


def max_variance_rows(seed, count):
    """Adversarial values: every V element 0.45-0.55 fp16 ulp above a grid point in [4, 5) (the largest
    stochastic-rounding variance, ulp^2 / 4, in every dimension), with 8-200 keys aligned with the query carrying most
    of the weight. sqrt(var), built from the largest |v| and a bound u^2 x^2 on each rounding's variance, is then
    tight, and the largest of a row's dimensions can exceed 1.5 sqrt(var)."""
    rng = np.random.default_rng(seed)
    for i in range(count):
        hd = (64, 128)[i % 2]
        n = int(rng.choice([300, 1000, 2048]))
        q = rng.standard_normal(hd)
        k = rng.standard_normal((n, hd))
        m = rng.integers(0, 256, (n, hd))
        v = rng.choice([-1, 1], (n, hd)) * (4 + (m + 0.5 + rng.uniform(-0.05, 0.05, (n, hd))) / 256)
        neff = int(rng.choice([8, 12, 16, 24, 32, 64, 200]))
        hot = rng.choice(n, neff, replace=False)
        k[hot] = q / np.linalg.norm(q) * np.sqrt(hd) * 1.5 + 0.3 * rng.standard_normal((neff, hd))
        yield q, k, v


def test_values_at_the_largest_rounding_variance_are_the_estimates_limit():
    """The estimate's documented limit, pinned: on max_variance_rows rows the estimate keeps err by at most 1.25e-3
    (measured: 4 of 300 kept rows over the bar, the worst 1.18e-3; rounding to nearest keeps 33 over it). Callers
    that need the bar for such data use the fp32 route."""
    worst_kept, over, over_rn = 0.0, 0, 0
    for q, k, v in max_variance_rows(7, 300):
        err, qh, p, l, o = emulate(q, k, v)
        if kept(estimate(qh, k, v, p, l, o)):
            worst_kept = max(worst_kept, err)
            over += err > BUDGET
        err0, qh, p, l, o = emulate(q, k, v, sr=False)
        over_rn += kept(estimate(qh, k, v, p, l, o, sr=False)) and err0 > BUDGET
    print(f"kept rows over the bar: {over} (worst {worst_kept:.2e}); rounding to nearest: {over_rn}")
    assert worst_kept <= 1.25e-3 and over <= 6 and over_rn > over


def test_flat_scores_with_correlated_values():
    """Rows whose scores span less than one fp16 step of the weights (a query scaled by 1e-4 .. 3e-2: nearly uniform
    attention) over K and V from shared rank-1/2 hidden states, values scaled to |v| <= 2-10. Below q x 1e-3 every
    weight rounds to the same fp16 value and the scores' differences are lost: the flatness test catches exactly
    those rows (recomputed). Above it the weights' rounding is still a monotone function of the score and
    correlates with V, so the error outgrows sqrt(var) (measured up to 3.4x), but it stays small in absolute terms:
    rows the kernel keeps err by at most 4e-4."""
    rng = np.random.default_rng(9)
    worst_kept, n_flat = 0.0, 0
    for i in range(200):
        hd = (64, 128)[i % 2]
        n = int(rng.choice([300, 1000, 4096]))
        q, k, v = correlated(rng, n, hd, int(rng.choice([1, 2])), 1.0, 1.0, False)
        qs = float(rng.choice([1e-4, 3e-4, 1e-3, 3e-3, 1e-2, 3e-2]))
        q = q * qs
        v = v * (2 * float(rng.choice([1.0, 3.0, 5.0])) / max(float(np.abs(v).max()), 1e-9))
        err, qh, p, l, o = emulate(q, k, v)
        if flat_row(p):
            n_flat += 1
        elif kept(estimate(qh, k, v, p, l, o)):
            worst_kept = max(worst_kept, err)
        if qs <= 1e-4:
            assert flat_row(p), (qs, n)
    assert worst_kept <= 4e-4, worst_kept
    assert n_flat > 0


def test_flatness_test_spares_ordinary_rows(cases):
    """The flatness test flags no row of the ordinary families (N(0,1), outliers, correlated hidden states): their
    weights are far from equal."""
    assert not any(flat_row(c[9]) for c in cases)
