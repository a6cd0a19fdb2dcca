"""CPU pins of the device sketch's schedule (ferrisboost_amd/csrc/fbhip_sketch.hip).

The device reorganises FeatureSketch (src/data/sketch.rs:72-302) in two ways:

* the binary counter's merges run level by level: block k of 2^(l+1) batches
  is merge(block 2k, block 2k + 1) of level l, compressed; collapse() then
  merges the blocks left at the set bits of the batch count, lowest level
  first, and compresses once;
* compress()'s greedy walk (:404-440) runs as a prefix maximum:
  taken_k = k + min(n - slots, max(0, max_{i<=k} (lb_i - i))), lb_k the first
  index >= 1 whose rmid reaches target_k, found from the entries' side (entry
  i takes the k with c_{i-1} < k <= c_i, c_i the targets its rmid reaches).

This file models both in f32 numpy arithmetic and checks, on small inputs
with many batches, that they give the host sketch's cuts bit for bit (the
product's fbt_sketch_cuts and the oracle's sketch), and that the prefix form
equals the walk on the summaries the sketch produces. The GPU suite checks
the kernels themselves against the same cuts.
"""

from __future__ import annotations

import numpy as np
import pytest

f32 = np.float32


def _summary(vals):
    """build_summary of one batch, unit weights, in the device's key order
    (both zeros one key; the zero entry is -0.0 when every zero is)."""
    u = vals.view(np.uint32).copy()
    u[(u & 0x7FFFFFFF) == 0] = 0
    keys = np.sort(u.astype(np.uint64) ^ np.where(u >> 31, 0xFFFFFFFF, 0x80000000).astype(np.uint64))
    zeros = vals[vals == 0]
    neg_only = zeros.size > 0 and bool(np.signbit(zeros).all())
    out = []
    i = 0
    n = len(keys)
    while i < n:
        j = i
        while j + 1 < n and keys[j + 1] == keys[i]:
            j += 1
        k = int(keys[i])
        u = (k & 0x7FFFFFFF) if k & 0x80000000 else (~k & 0xFFFFFFFF)
        v = np.array([u], np.uint32).view(np.float32)[0]
        if v == 0 and neg_only:
            v = f32(-0.0)
        out.append([v, f32(j + 1 - i), f32(i), f32(j + 1)])
        i = j + 1
    return out


def _merge(a, b):
    out = []
    i = j = 0
    pa = pb = f32(0.0)
    while i < len(a) or j < len(b):
        ta = j >= len(b) or (i < len(a) and a[i][0] <= b[j][0])
        if ta:
            e = a[i]
            out.append([e[0], e[1], f32(e[2] + pb), f32(e[3] + pb)])
            pa = e[3]
            i += 1
        else:
            e = b[j]
            out.append([e[0], e[1], f32(e[2] + pa), f32(e[3] + pa)])
            pb = e[3]
            j += 1
    ded = []
    for e in out:
        if ded and ded[-1][0] == e[0]:
            ded[-1][1] = f32(ded[-1][1] + e[1])
            ded[-1][2] = min(ded[-1][2], e[2])
            ded[-1][3] = max(ded[-1][3], e[3])
        else:
            ded.append(list(e))
    return ded


def _mid(e):
    return f32(f32(0.5) * f32(e[2] + e[3]))


def _compress_walk(s, cap):
    n = len(s)
    if n <= cap:
        return s
    total = s[-1][3]
    slots = cap - 1
    out = [s[0]]
    last = 0
    for k in range(1, slots):
        target = f32(f32(total * f32(k)) / f32(slots))
        j = last + 1
        while j < n - 1 and _mid(s[j]) < target:
            j += 1
        j = min(max(j, last + 1), n - 1 - (slots - 1 - k))
        if j > last:
            out.append(s[j])
            last = j
    if last < n - 1:
        out.append(s[-1])
    return out


def _compress_prefix(s, cap):
    n = len(s)
    if n <= cap:
        return s
    total = s[-1][3]
    slots = cap - 1
    mids = [_mid(e) for e in s]
    out = [s[0]]
    run = -(1 << 30)
    taken = 0
    for k in range(1, slots):
        target = f32(f32(total * f32(k)) / f32(slots))
        lb = next((i for i in range(1, n - 1) if mids[i] >= target), n - 1)
        run = max(run, lb - k)
        taken = k + min(n - slots, max(0, run))
        out.append(s[taken])
    if taken < n - 1:
        out.append(s[-1])
    return out


def _compress_scatter(s, cap):
    """The device's compress: lb from the entries' side (entry i takes the
    targets k in (c_{i-1}, c_i], c_i = the targets its rmid reaches), then
    the prefix maximum."""
    n = len(s)
    if n <= cap:
        return s
    total = s[-1][3]
    slots = cap - 1

    def target(k):
        return f32(f32(total * f32(k)) / f32(slots))

    def upto(m):
        k = min(max(int(float(m) * slots / float(total)), 0), slots - 1)
        while k + 1 <= slots - 1 and target(k + 1) <= m:
            k += 1
        while k >= 1 and target(k) > m:
            k -= 1
        return k

    lb = [n - 1] * slots
    for i in range(1, n - 1):
        lo = 0 if i == 1 else upto(_mid(s[i - 1]))
        for k in range(lo + 1, upto(_mid(s[i])) + 1):
            lb[k] = i
    out = [s[0]]
    run = -(1 << 30)
    taken = 0
    for k in range(1, slots):
        run = max(run, lb[k] - k)
        taken = k + min(n - slots, max(0, run))
        out.append(s[taken])
    if taken < n - 1:
        out.append(s[-1])
    return out


def _midpoint(a, b):
    d = f32(b - a)
    m = f32(a + f32(d * f32(0.5))) if np.isfinite(d) else f32(f32(a * f32(0.5)) + f32(b * f32(0.5)))
    return b if m <= a else m


def _device_cuts(col, max_bin, compress=_compress_scatter):
    """The device's schedule for one numeric feature (unit weights)."""
    n_cuts = max_bin - 1
    if n_cuts <= 0:
        return []
    cap = max(16 * max_bin, 32)
    vals = col[~np.isnan(col)].astype(np.float32)
    m = (len(vals) + cap - 1) // cap
    if m == 0:
        return []
    level = [_summary(vals[k * cap:(k + 1) * cap]) for k in range(m)]
    held = {}
    lv = 0
    while level:
        if len(level) % 2:
            held[lv] = level[-1]
        level = [compress(_merge(level[2 * k], level[2 * k + 1]), cap)
                 for k in range(len(level) // 2)]
        lv += 1
    acc = None
    for l in sorted(held):
        acc = held[l] if acc is None else _merge(acc, held[l])
    s = compress(acc, cap)
    if len(s) <= n_cuts:
        return [_midpoint(s[i][0], s[i + 1][0]) for i in range(len(s) - 1)]
    total = s[-1][3]
    mids = [_mid(e) for e in s]
    out = []
    for k in range(1, n_cuts + 1):
        target = f32(f32(total * f32(k)) / f32(max_bin))
        idx = next((i for i in range(len(s)) if not mids[i] < target), len(s))
        v = s[min(idx, len(s) - 1)][0]
        if not out or v > out[-1]:
            out.append(v)
    return out


def _columns(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 3000))
    cols = [
        rng.standard_normal(n).astype(np.float32),
        rng.integers(0, 7, n).astype(np.float32),                  # few distinct values
        rng.integers(0, 300, n).astype(np.float32),                # ties across batches
        np.round(rng.standard_normal(n) * 4).astype(np.float32),   # heavy duplicates, both zeros
        np.where(rng.random(n) < 0.3, np.round(rng.standard_normal(n)) * 0.0,
                 rng.standard_normal(n)).astype(np.float32),       # a mass of both zeros
        np.where(rng.random(n) < 0.3, np.nan, rng.random(n)).astype(np.float32),
        np.where(rng.random(n) < 0.05, np.inf, rng.standard_exponential(n)).astype(np.float32),
    ]
    return np.stack(cols, axis=1)


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("max_bin", [2, 3, 4, 16])
def test_level_schedule_and_prefix_compress_give_the_host_cuts(oracle, seed, max_bin):
    from ferrisboost_amd import _native as N

    x = np.ascontiguousarray(_columns(seed))
    n, nf = x.shape
    vals, offs = oracle.sketch_cuts(x, max_bin)
    pv = np.zeros(max(1, nf * 65536), np.float32)
    po = np.zeros(nf + 1, np.uint32)
    N.check_train(N.train_lib().fbt_sketch_cuts(N.ptr(x), n, nf, max_bin, None, None,
                                                N.ptr(pv), N.ptr(po)))
    for f in range(nf):
        want = vals[offs[f]:offs[f + 1]]
        assert np.array_equal(pv[po[f]:po[f + 1]].view(np.uint32), want.view(np.uint32))
        got = np.array(_device_cuts(x[:, f], max_bin), np.float32)
        z = x[:, f][x[:, f] == 0]
        if np.signbit(z).any() and not np.signbit(z).all() and (got == 0).any():
            # the one undecided case: the zero cut's sign follows the host's sort
            assert np.array_equal(got, want)
            continue
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (seed, max_bin, f)


def test_prefix_compress_equals_the_walk_on_sketch_summaries():
    """compress as a prefix maximum equals the walk entry for entry, on the
    merged summaries a sketch builds (duplicates, NaNs dropped, many batches)."""
    rng = np.random.default_rng(7)
    checked = 0
    for trial in range(40):
        cap = int(rng.choice([32, 48, 64]))
        a = _summary((np.round(rng.standard_normal(cap) * rng.choice([2, 50])) + 0.0).astype(np.float32))
        b = _summary((np.round(rng.standard_normal(cap) * rng.choice([2, 50])) + 0.0).astype(np.float32))
        for _ in range(3):
            m = _merge(a, b)
            if len(m) > cap:
                checked += 1
            w = _compress_walk(m, cap)
            p = _compress_prefix(m, cap)
            q = _compress_scatter(m, cap)
            assert [list(map(float, e)) for e in w] == [list(map(float, e)) for e in p], trial
            assert [list(map(float, e)) for e in w] == [list(map(float, e)) for e in q], trial
            a, b = w, _summary((np.round(rng.standard_normal(cap) * 9) + 0.0).astype(np.float32))
    assert checked > 20
