// fbhip_sketch.hip -- the quantile sketch of DenseSource on the device
// (SketchSet::with_categorical / push_row / finalize_checked,
// src/data/sketch.rs:440-560, over FeatureSketch, :72-302).
//
// FeatureSketch feeds a numeric feature's non-missing values, in row order,
// into batches of limit = max(16 max_bins, 32) values. A full batch (and at
// the end the partial one) becomes a sorted summary of its distinct values,
// each with its weight and rank interval [rmin, rmax] (build_summary,
// :305-327). Summaries go into a binary counter of levels: a summary meeting
// an occupied level merges with it, older one first (merge_entries +
// dedup_same_value, :334-400), is compressed back to `limit` entries
// (compress, :404-440) and moves up a level (insert_level, :148-171).
// cuts() merges what the levels hold, lowest level first, compresses once
// and picks max_bins - 1 values (collapse + cuts, :172-271).
//
// With unit row weights every step is a fixed function of the values in row
// order, so the device reproduces each summary entry for entry:
//   * compaction: each feature's non-missing values in row order, from
//     staged row-major chunks (a count pass, then ranks by wave ballots);
//   * batch summaries: one workgroup sorts a batch in LDS (bitonic, on
//     order-preserving integer keys) and writes one entry per distinct
//     value, rank interval [first index, last index + 1): the host's running
//     f32 sums are those integers exactly (a batch holds at most 16384);
//   * the counter's merges level by level, the merges of a level in
//     parallel (block k of 2^(l+1) batches merges blocks 2k and 2k + 1 of
//     level l, which is the order in which the counter meets them), each
//     with a merge-path split of the output, equal values combined, and the
//     compression as a prefix maximum (sk_merge_kernel);
//   * the final merges and the cut choice, one workgroup per feature.
// Entries combine with the same f32 operations in the same order, so the
// cuts equal the host sketch's bit for bit. -0.0 and +0.0 compare equal, so
// they form one entry on both sides and the rank arithmetic never sees the
// sign; the entry's value takes the sign of whichever zero the host's
// unstable sort put first. The device gives a batch's zero entry the sign
// its zeros share (+0.0 when they differ), so only a feature holding both
// signs whose cuts include a zero can differ: it is reported, and the
// caller sketches it on the host.
// Categorical features only need their largest code and the first invalid
// value (FeatureSketch::push, :121-131), reduced while the rows are staged.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/fbhip.h"
#include "fbhip_internal.h"

using namespace fbh;

namespace {

struct SkError : std::runtime_error {
    int code;
    SkError(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

void sk_check(hipError_t e, const char *what) {
    if (e != hipSuccess)
        throw SkError(FBH_RUNTIME_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}

template <class F>
int sk_guard(F &&f) {
    try {
        f();
        return FBH_OK;
    } catch (const SkError &e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::exception &e) {
        set_last_error(e.what());
        return FBH_RUNTIME_ERROR;
    }
}

// A summary entry (Entry, src/data/sketch.rs:35-46).
struct SkEntry {
    float v, w, rmin, rmax;
};

constexpr uint32_t SK_TPB = 256;
constexpr uint32_t SK_ROWS = 64;   // rows of a staging tile (one wave of lanes)
constexpr uint32_t SK_FEATS = 64;  // features of a staging tile
constexpr uint32_t SK_MAX_BIN = 1024;                   // largest max_bin sketched here
constexpr uint64_t SK_STAGE_BYTES = 256ull << 20;      // row staging of one chunk

__host__ __device__ inline uint32_t sk_limit(uint32_t max_bin) {
    const uint32_t l = 16u * max_bin;
    return l > 32u ? l : 32u;
}

// Order-preserving integer key; both zeros take +0.0's key (they compare
// equal on the host).
constexpr uint32_t SK_ZERO_KEY = 0x80000000u;

__device__ __forceinline__ uint32_t sk_key(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) == 0) u = 0;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float sk_unkey(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ SkEntry sk_ld(const SkEntry *p) {
    const float4 q = *reinterpret_cast<const float4 *>(p);
    return SkEntry{q.x, q.y, q.z, q.w};
}

__device__ __forceinline__ void sk_st(SkEntry *p, const SkEntry &e) {
    *reinterpret_cast<float4 *>(p) = make_float4(e.v, e.w, e.rmin, e.rmax);
}

// Entry::rmid (src/data/sketch.rs:43-45).
__device__ __forceinline__ float sk_mid(const SkEntry *p) {
    const float2 r = *reinterpret_cast<const float2 *>(&p->rmin);
    return 0.5f * (r.x + r.y);
}

// midpoint (src/data/sketch.rs:290-302); no contraction (the file is built
// with -ffp-contract=off), so a + d * 0.5 rounds twice, as on the host.
__device__ __forceinline__ float sk_midpoint(float a, float b) {
    const float d = b - a;
    const float m = isfinite(d) ? a + d * 0.5f : a * 0.5f + b * 0.5f;
    return m <= a ? b : m;
}

// Exclusive sum over the block (blockDim.x == SK_TPB); buf holds 8 entries.
__device__ uint32_t sk_scan_sum(uint32_t v, uint32_t *buf, uint32_t &total) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t t = __shfl_up(incl, off, 64);
        if (lane >= (uint32_t)off) incl += t;
    }
    __syncthreads();
    if (lane == 63) buf[wave] = incl;
    __syncthreads();
    uint32_t before = 0, tot = 0;
    for (uint32_t w = 0; w < SK_TPB / 64; w++) {
        if (w < wave) before += buf[w];
        tot += buf[w];
    }
    total = tot;
    return before + incl - v;
}

// Exclusive maximum over the block (INT_MIN for thread 0); buf holds 8.
__device__ int sk_scan_max(int v, int *buf) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off, 64);
        if (lane >= (uint32_t)off) incl = max(incl, t);
    }
    __syncthreads();
    if (lane == 63) buf[wave] = incl;
    __syncthreads();
    int before = INT_MIN;
    for (uint32_t w = 0; w < wave; w++) before = max(before, buf[w]);
    int excl = __shfl_up(incl, 1, 64);
    if (lane == 0) excl = INT_MIN;
    return max(before, excl);
}

// ---------------------------------------------------------------- staging

// One 64-row x 64-feature tile of a staged row-major chunk, transposed
// through LDS so that a wave holds one feature's 64 rows (lane = row).
__device__ __forceinline__ void sk_load_tile(float (*blk)[SK_FEATS + 1], const float *x,
                                             uint64_t n_rows, uint32_t nf, uint64_t rb,
                                             uint32_t fb) {
    const uint32_t nr = (uint32_t)min<uint64_t>(SK_ROWS, n_rows - rb);
    const uint32_t nfb = min(SK_FEATS, nf - fb);
    for (uint32_t i = threadIdx.x; i < SK_ROWS * SK_FEATS; i += SK_TPB) {
        const uint32_t r = i / SK_FEATS, f = i % SK_FEATS;
        if (f < nfb) blk[r][f] = r < nr ? x[(rb + r) * nf + fb + f] : __uint_as_float(0x7FC00000u);
    }
    __syncthreads();
}

// Per tile: non-missing counts of every numeric feature (cnt[tile row][j]),
// the zero signs seen (bit 0: -0.0, bit 1: +0.0), and for categorical
// features the largest valid code and whether an invalid one occurred
// (categorical::invalid_code: negative, above 65533 or fractional).
__global__ __launch_bounds__(SK_TPB) void sk_count_kernel(
    const float *__restrict__ x, uint64_t n_rows, uint32_t nf, const int32_t *__restrict__ num_of,
    uint32_t n_num, uint32_t *__restrict__ cnt, uint32_t *__restrict__ zero,
    int32_t *__restrict__ cat_max, uint32_t *__restrict__ cat_bad) {
    __shared__ float blk[SK_ROWS][SK_FEATS + 1];
    const uint64_t rb = (uint64_t)blockIdx.x * SK_ROWS;
    const uint32_t fb = blockIdx.y * SK_FEATS;
    sk_load_tile(blk, x, n_rows, nf, rb, fb);
    const uint32_t nfb = min(SK_FEATS, nf - fb);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    for (uint32_t f = wave; f < nfb; f += SK_TPB / 64) {
        const float v = blk[lane][f];
        const bool valid = !(v != v);
        const int32_t j = num_of[fb + f];
        if (j >= 0) {
            const uint64_t m = __ballot(valid);
            const uint64_t neg = __ballot(valid && v == 0.0f && signbit(v));
            const uint64_t pos = __ballot(valid && v == 0.0f && !signbit(v));
            if (lane == 0) {
                cnt[(uint64_t)blockIdx.x * n_num + j] = (uint32_t)__popcll(m);
                const uint32_t z = (neg ? 1u : 0u) | (pos ? 2u : 0u);
                if (z) atomicOr(&zero[j], z);
            }
        } else {
            const bool bad = valid && (v < 0.0f || v > 65533.0f || v != truncf(v));
            int code = valid && !bad ? (int)v : -1;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) code = max(code, __shfl_xor(code, off, 64));
            const uint64_t b = __ballot(bad);
            if (lane == 0) {
                if (code >= 0) atomicMax(&cat_max[fb + f], code);
                if (b) atomicOr(&cat_bad[fb + f], 1u);
            }
        }
    }
}

// Per numeric feature j: off[tile row][j] = n_valid[j] + the counts of the
// chunk's earlier tile rows; n_valid[j] then grows by the chunk's count.
__global__ __launch_bounds__(SK_TPB) void sk_offsets_kernel(const uint32_t *__restrict__ cnt,
                                                            uint32_t n_tiles, uint32_t n_num,
                                                            uint32_t *__restrict__ off,
                                                            uint64_t *__restrict__ n_valid) {
    __shared__ uint32_t buf[8];
    const uint32_t j = blockIdx.x;
    uint64_t carry = n_valid[j];
    for (uint32_t t0 = 0; t0 < n_tiles; t0 += SK_TPB) {
        const uint32_t t = t0 + threadIdx.x;
        const uint32_t c = t < n_tiles ? cnt[(uint64_t)t * n_num + j] : 0u;
        uint32_t total;
        const uint32_t before = sk_scan_sum(c, buf, total);
        // Offsets within a feature stay below 2^32: the sketch holds at most
        // 2^32 - 1 rows.
        if (t < n_tiles) off[(uint64_t)t * n_num + j] = (uint32_t)(carry + before);
        carry += total;
    }
    if (threadIdx.x == 0) n_valid[j] = carry;
}

// Each numeric feature's non-missing values of the chunk, in row order, at
// their offsets of comp[j * stride ..].
__global__ __launch_bounds__(SK_TPB) void sk_compact_kernel(
    const float *__restrict__ x, uint64_t n_rows, uint32_t nf, const int32_t *__restrict__ num_of,
    uint32_t n_num, const uint32_t *__restrict__ off, float *__restrict__ comp, uint64_t stride) {
    __shared__ float blk[SK_ROWS][SK_FEATS + 1];
    const uint64_t rb = (uint64_t)blockIdx.x * SK_ROWS;
    const uint32_t fb = blockIdx.y * SK_FEATS;
    sk_load_tile(blk, x, n_rows, nf, rb, fb);
    const uint32_t nfb = min(SK_FEATS, nf - fb);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (uint32_t f = wave; f < nfb; f += SK_TPB / 64) {
        const int32_t j = num_of[fb + f];
        if (j < 0) continue;
        const float v = blk[lane][f];
        const bool valid = !(v != v);
        const uint64_t m = __ballot(valid);
        if (valid) {
            const uint32_t pos = off[(uint64_t)blockIdx.x * n_num + j] + (uint32_t)__popcll(m & below);
            comp[(uint64_t)j * stride + pos] = v;
        }
    }
}

// ---------------------------------------------------------------- summaries

// One batch: len values (at most the padded size P, a power of two, of the
// dynamic LDS keys) into dst, one entry per distinct value; *n_dst = the
// entry count.
struct SkSortTask {
    const float *src;
    SkEntry *dst;
    uint32_t *n_dst;
    uint32_t len;
    uint32_t pad;
};

__global__ __launch_bounds__(SK_TPB) void sk_sort_kernel(const SkSortTask *__restrict__ tasks,
                                                         uint32_t P) {
    extern __shared__ uint32_t keys[];
    __shared__ uint32_t buf[8];
    __shared__ uint32_t zsigns;  // bit 0: a -0.0 seen, bit 1: a +0.0 seen
    const SkSortTask T = tasks[blockIdx.x];
    const uint32_t len = T.len;
    if (threadIdx.x == 0) zsigns = 0;
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < P; i += SK_TPB) {
        uint32_t k = 0xFFFFFFFFu;
        if (i < len) {
            const float v = T.src[i];
            k = sk_key(v);
            if (k == SK_ZERO_KEY) atomicOr(&zsigns, signbit(v) ? 1u : 2u);
        }
        keys[i] = k;
    }
    __syncthreads();
    // Bitonic sort, ascending.
    for (uint32_t k = 2; k <= P; k <<= 1) {
        for (uint32_t s = k >> 1; s > 0; s >>= 1) {
            for (uint32_t i = threadIdx.x; i < P / 2; i += SK_TPB) {
                const uint32_t lo = 2 * i - (i & (s - 1)), hi = lo + s;
                const uint32_t a = keys[lo], b = keys[hi];
                const bool asc = (lo & k) == 0;
                if ((a > b) == asc) {
                    keys[lo] = b;
                    keys[hi] = a;
                }
            }
            __syncthreads();
        }
    }
    // build_summary: the entry of a run of equal keys [s, e] is written by the
    // thread holding e, at the run's index among runs.
    const uint32_t per = (len + SK_TPB - 1) / SK_TPB;
    const uint32_t p0 = min(len, threadIdx.x * per), p1 = min(len, p0 + per);
    uint32_t ends = 0;
    for (uint32_t p = p0; p < p1; p++) ends += (p + 1 == len || keys[p + 1] != keys[p]) ? 1u : 0u;
    uint32_t total;
    uint32_t g = sk_scan_sum(ends, buf, total);
    for (uint32_t p = p0; p < p1; p++) {
        if (!(p + 1 == len || keys[p + 1] != keys[p])) continue;
        const uint32_t key = keys[p];
        uint32_t lo = 0, hi = p;  // first index holding key
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (keys[mid] < key) lo = mid + 1;
            else hi = mid;
        }
        const float v = key == SK_ZERO_KEY && zsigns == 1u ? -0.0f : sk_unkey(key);
        sk_st(T.dst + g, SkEntry{v, (float)(p + 1 - lo), (float)lo, (float)(p + 1)});
        g++;
    }
    if (threadIdx.x == 0) *T.n_dst = total;
}

// ---------------------------------------------------------------- merges

// merge_entries(a, b) + dedup_same_value into d, then, when `prune` and the
// result holds more than `limit` entries, compress(d, limit) in place.
struct SkMergeTask {
    const SkEntry *a;
    const SkEntry *b;
    SkEntry *d;
    const uint32_t *na;
    const uint32_t *nb;
    uint32_t *nd;
};

// compress's targets: target_k = total * k / slots (f32, two roundings).
__device__ __forceinline__ float sk_target(float total, uint32_t k, uint32_t slots) {
    return total * (float)k / (float)slots;
}

// The largest k in [0, slots - 1] with target_k <= m (0: none). The targets
// never decrease in k, so an estimate from the exact quotient is moved to
// the boundary by evaluating the targets themselves.
__device__ uint32_t sk_targets_upto(float m, float total, uint32_t slots) {
    const double e = (double)m * (double)slots / (double)total;
    uint32_t k = e <= 0.0 ? 0u : (e >= (double)(slots - 1) ? slots - 1 : (uint32_t)e);
    while (k + 1 <= slots - 1 && sk_target(total, k + 1, slots) <= m) k++;
    while (k >= 1 && sk_target(total, k, slots) > m) k--;
    return k;
}

// compress as a prefix maximum. The host walk keeps entry 0, then for
// k = 1 .. slots - 1 the first j >= taken + 1 whose rmid reaches target_k
// (stopping at n - 1), capped at n - 1 - (slots - 1 - k), and finally entry
// n - 1 if not taken. rmid never decreases along a summary (every entry's
// rmin is at least its predecessor's rmax, and f32 rounding is monotone), so
// the walk's j is max(taken + 1, lb_k), lb_k = the first index in
// [1, n - 2] whose rmid reaches target_k (n - 1 if none). With
// u_k = taken_k - k the recurrence becomes
// u_k = min(max(lb_k - k, u_{k-1}), n - slots), u_0 = 0, that is
// taken_k = k + min(n - slots, max(0, max_{i <= k} (lb_i - i))).
// lb comes from the entries' side: with c_i the number of targets entry i's
// rmid reaches (nondecreasing in i), lb_k = i for c_{i-1} < k <= c_i
// (c_0 = 0), so each entry scatters its own k and the reads are coalesced.
// Writes taken_k into sel[k] for k = 1 .. slots - 1; every thread calls it.
template <class IDX>
__device__ void sk_compress_plan(const SkEntry *s, uint32_t n, uint32_t slots, IDX *sel,
                                 int *ibuf) {
    const float total = s[n - 1].rmax;
    for (uint32_t k = 1 + threadIdx.x; k < slots; k += SK_TPB) sel[k] = (IDX)(n - 1);
    __syncthreads();
    for (uint32_t i = 1 + threadIdx.x; i + 1 < n; i += SK_TPB) {
        const uint32_t ci = sk_targets_upto(sk_mid(s + i), total, slots);
        const uint32_t cp = i == 1 ? 0u : sk_targets_upto(sk_mid(s + i - 1), total, slots);
        for (uint32_t k = cp + 1; k <= ci; k++) sel[k] = (IDX)i;
    }
    __syncthreads();
    const uint32_t nk = slots - 1;
    const uint32_t per = (nk + SK_TPB - 1) / SK_TPB;
    const uint32_t ka = 1 + min(nk, threadIdx.x * per), kb = 1 + min(nk, threadIdx.x * per + per);
    int run = INT_MIN;
    for (uint32_t k = ka; k < kb; k++) run = max(run, (int)sel[k] - (int)k);
    int r = sk_scan_max(run, ibuf);
    const int C = (int)(n - slots);
    for (uint32_t k = ka; k < kb; k++) {
        r = max(r, (int)sel[k] - (int)k);
        sel[k] = (IDX)(k + (uint32_t)min(C, max(0, r)));
    }
    __syncthreads();
}

// Merge path: the a-entries among the first k outputs of merge(a, b) (on
// equal values a's entry goes first).
__device__ uint32_t sk_merge_path(const SkEntry *a, uint32_t na, const SkEntry *b, uint32_t nb,
                                  uint32_t k) {
    uint32_t lo = k > nb ? k - nb : 0u, hi = min(k, na);
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (a[mid].v <= b[k - mid - 1].v) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// The merged output runs in chunks of SK_MCH: each chunk's entries of a and
// b (plus one on each side) are staged in LDS with coalesced loads, each
// thread merges SK_MPT outputs from there, and the runs of equal values are
// counted by a block scan. Chunk boundaries come from one merge-path search
// each, all at once.
constexpr uint32_t SK_MCH = 1024;
constexpr uint32_t SK_MPT = SK_MCH / SK_TPB;
constexpr uint32_t SK_MAX_CHUNKS = 64;  // 2 * 16 * 1024 outputs at most under `prune`

__global__ __launch_bounds__(SK_TPB) void sk_merge_kernel(const SkMergeTask *__restrict__ tasks,
                                                          uint32_t limit, uint32_t prune) {
    extern __shared__ uint16_t sel[];
    __shared__ SkEntry sa[SK_MCH + 2], sb[SK_MCH + 2];
    __shared__ uint32_t bound[SK_MAX_CHUNKS + 1];
    __shared__ uint32_t buf[8];
    __shared__ int ibuf[8];
    const SkMergeTask T = tasks[blockIdx.x];
    const SkEntry *a = T.a, *b = T.b;
    const uint32_t na = *T.na, nb = *T.nb, M = na + nb;
    const uint32_t n_ch = (M + SK_MCH - 1) / SK_MCH;
    uint32_t out = 0;  // entries written so far
    for (uint32_t g0 = 0; g0 < n_ch; g0 += SK_MAX_CHUNKS) {
        // Boundaries of chunks g0 .. g0 + SK_MAX_CHUNKS (a-entries before each).
        const uint32_t gn = min(SK_MAX_CHUNKS, n_ch - g0);
        for (uint32_t t = threadIdx.x; t <= gn; t += SK_TPB)
            bound[t] = sk_merge_path(a, na, b, nb, min(M, (g0 + t) * SK_MCH));
        __syncthreads();
        for (uint32_t g = 0; g < gn; g++) {
            const uint32_t c0 = (g0 + g) * SK_MCH, c1 = min(M, c0 + SK_MCH);
            const uint32_t ia = bound[g], jb = c0 - ia, ia1 = bound[g + 1], jb1 = c1 - ia1;
            // sa[x] = a[ia - 1 + x] for x in [0, ia1 - ia + 2), where present.
            for (uint32_t x = threadIdx.x; x < ia1 - ia + 2; x += SK_TPB) {
                const uint32_t i = ia + x;  // a[i - 1]
                if (i >= 1 && i - 1 < na) sa[x] = sk_ld(a + i - 1);
            }
            for (uint32_t x = threadIdx.x; x < jb1 - jb + 2; x += SK_TPB) {
                const uint32_t j = jb + x;
                if (j >= 1 && j - 1 < nb) sb[x] = sk_ld(b + j - 1);
            }
            __syncthreads();
            // This thread's outputs [k0, k1) of the chunk.
            const uint32_t len = c1 - c0, la = ia1 - ia, lb = jb1 - jb;
            const uint32_t k0 = min(len, threadIdx.x * SK_MPT), k1 = min(len, k0 + SK_MPT);
            uint32_t il;
            {
                uint32_t lo = k0 > lb ? k0 - lb : 0u, hi = min(k0, la);
                while (lo < hi) {
                    const uint32_t mid = (lo + hi) >> 1;
                    if (sa[mid + 1].v <= sb[k0 - mid].v) lo = mid + 1;
                    else hi = mid;
                }
                il = lo;
            }
            uint32_t i = ia + il, j = jb + (k0 - il);  // global positions
#define SA(q) sa[(q) - ia + 1]
#define SB(q) sb[(q) - jb + 1]
            const uint32_t kk = c0 + k0;  // global output index
            bool has_prev = kk > 0;
            float prev = 0.0f;
            if (has_prev) {
                if (i == 0) prev = SB(j - 1).v;
                else if (j == 0) prev = SA(i - 1).v;
                else prev = fmaxf(SA(i - 1).v, SB(j - 1).v);
            }
            float pa = i > 0 ? SA(i - 1).rmax : 0.0f;  // pass_a: rmax of a's last entry taken
            float pb = j > 0 ? SB(j - 1).rmax : 0.0f;
            SkEntry e[SK_MPT];
            uint32_t flags = 0;  // bit q: output k0 + q starts a run
#pragma unroll
            for (uint32_t q = 0; q < SK_MPT; q++) {
                e[q] = SkEntry{};
                if (k0 + q < k1) {
                    const bool ta = i < na && (j >= nb || SA(i).v <= SB(j).v);
                    SkEntry x = ta ? SA(i) : SB(j);
                    const float sh = ta ? pb : pa;
                    const float xr = x.rmax;
                    x.rmin = x.rmin + sh;
                    x.rmax = x.rmax + sh;
                    if (ta) {
                        pa = xr;
                        i++;
                    } else {
                        pb = xr;
                        j++;
                    }
                    const bool start = !has_prev || x.v != prev;
                    prev = x.v;
                    has_prev = true;
                    // A run's partner (the other summary's entry of the same
                    // value) is always the next output; staged, since
                    // outputs up to c1 are.
                    if (start && kk + q + 1 < M) {
                        const bool ta2 = i < na && (j >= nb || SA(i).v <= SB(j).v);
                        const SkEntry y = ta2 ? SA(i) : SB(j);
                        if (y.v == x.v) {
                            const float sh2 = ta2 ? pb : pa;
                            x.w = x.w + y.w;
                            x.rmin = fminf(x.rmin, y.rmin + sh2);
                            x.rmax = fmaxf(x.rmax, y.rmax + sh2);
                        }
                    }
                    e[q] = x;
                    flags |= start ? 1u << q : 0u;
                }
            }
#undef SA
#undef SB
            uint32_t n_chunk;
            const uint32_t o = out + sk_scan_sum((uint32_t)__popc(flags), buf, n_chunk);
#pragma unroll
            for (uint32_t q = 0; q < SK_MPT; q++)
                if (flags >> q & 1u) sk_st(T.d + o + __popc(flags & ((1u << q) - 1u)), e[q]);
            out += n_chunk;
            __syncthreads();  // the staged entries are rewritten next
        }
    }
    const uint32_t n_out = out;
    if (!prune || n_out <= limit) {
        if (threadIdx.x == 0) *T.nd = n_out;
        return;
    }
    __syncthreads();  // d complete (global writes of one workgroup)
    // compress(d, limit) in place: entry k comes from sel[k] >= k, so the
    // reads of outputs 256 at a time precede the writes and never meet a
    // position already written.
    const uint32_t n = n_out, slots = limit - 1;
    const SkEntry last = sk_ld(T.d + n - 1);
    sk_compress_plan<uint16_t>(T.d, n, slots, sel, ibuf);
    for (uint32_t base = 1; base < slots; base += SK_TPB) {
        const uint32_t k = base + threadIdx.x;
        SkEntry v{};
        if (k < slots) v = sk_ld(T.d + sel[k]);
        __syncthreads();
        if (k < slots) sk_st(T.d + k, v);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        uint32_t c = slots;
        if (sel[slots - 1] < n - 1) sk_st(T.d + c++, last);
        *T.nd = c;
    }
}

// ---------------------------------------------------------------- cuts

// FeatureSketch::cuts over a feature's collapsed summary: compress it to
// `limit` entries into p when longer, then the cut values (at most
// max_bin - 1) into out and their count into *n_out.
struct SkCutTask {
    const SkEntry *all;
    const uint32_t *n_all;
    SkEntry *p;
    float *out;
    uint32_t *n_out;
    uint32_t pad[2];
};

__global__ __launch_bounds__(SK_TPB) void sk_cuts_kernel(const SkCutTask *__restrict__ tasks,
                                                         uint32_t limit, uint32_t max_bin) {
    extern __shared__ uint32_t lds[];
    uint32_t *sel = lds;                      // limit entries
    float *vals = reinterpret_cast<float *>(lds + limit);  // max_bin entries
    __shared__ uint32_t buf[8];
    __shared__ int ibuf[8];
    const SkCutTask T = tasks[blockIdx.x];
    const uint32_t n = *T.n_all;
    const SkEntry *s = T.all;
    uint32_t ns = n;
    if (n > limit) {
        const uint32_t slots = limit - 1;
        sk_compress_plan<uint32_t>(T.all, n, slots, sel, ibuf);
        for (uint32_t k = 1 + threadIdx.x; k < slots; k += SK_TPB) sk_st(T.p + k, sk_ld(T.all + sel[k]));
        if (threadIdx.x == 0) sk_st(T.p, sk_ld(T.all));
        ns = slots;
        if (sel[slots - 1] < n - 1) {
            if (threadIdx.x == 0) sk_st(T.p + slots, sk_ld(T.all + n - 1));
            ns = slots + 1;
        }
        s = T.p;
        __syncthreads();  // p complete
    }
    const uint32_t n_cuts = max_bin - 1;
    if (ns <= n_cuts) {  // low cardinality: midpoints of neighbours
        for (uint32_t i = threadIdx.x; i + 1 < ns; i += SK_TPB)
            T.out[i] = sk_midpoint(s[i].v, s[i + 1].v);
        if (threadIdx.x == 0) *T.n_out = ns ? ns - 1 : 0;
        return;
    }
    const float total = s[ns - 1].rmax;
    for (uint32_t k = 1 + threadIdx.x; k <= n_cuts; k += SK_TPB) {
        const float target = total * (float)k / (float)max_bin;
        uint32_t lo = 0, hi = ns;  // partition_point(rmid < target)
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (sk_mid(s + mid) < target) lo = mid + 1;
            else hi = mid;
        }
        vals[k - 1] = s[min(lo, ns - 1)].v;
    }
    __syncthreads();
    // The values never decrease in k; a value is kept when above the last
    // kept one, i.e. above its predecessor.
    const uint32_t per = (n_cuts + SK_TPB - 1) / SK_TPB;
    const uint32_t q0 = min(n_cuts, threadIdx.x * per), q1 = min(n_cuts, q0 + per);
    uint32_t keep = 0;
    for (uint32_t q = q0; q < q1; q++) keep += (q == 0 || vals[q] > vals[q - 1]) ? 1u : 0u;
    uint32_t kept;
    uint32_t o = sk_scan_sum(keep, buf, kept);
    for (uint32_t q = q0; q < q1; q++)
        if (q == 0 || vals[q] > vals[q - 1]) T.out[o++] = vals[q];
    if (threadIdx.x == 0) *T.n_out = kept;
}

uint32_t pow2_at_least(uint32_t v) {
    uint32_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

uint32_t bit_length(uint64_t v) {
    uint32_t b = 0;
    while (v) {
        b++;
        v >>= 1;
    }
    return b;
}

uint64_t stage_rows_of(uint64_t n_rows, uint32_t nf) {
    const uint64_t r = std::max<uint64_t>(SK_ROWS, SK_STAGE_BYTES / (4ull * std::max(nf, 1u)));
    return std::max<uint64_t>(1, std::min(n_rows, r));
}

// Device bytes of the sketch, with every value of every numeric feature
// non-missing (the largest case).
uint64_t sketch_bytes(uint64_t n_rows, uint32_t nf, uint32_t n_num, uint32_t max_bin) {
    const uint64_t stage = stage_rows_of(n_rows, nf);
    const uint64_t tiles = (stage + SK_ROWS - 1) / SK_ROWS;
    uint64_t b = 4 * stage * nf + 8 * tiles * n_num + 64ull * nf + (1u << 20);
    b += 4 * n_rows * n_num;  // compacted values
    if (max_bin >= 2) {
        const uint64_t L = sk_limit(max_bin);
        const uint64_t m = (n_rows + L - 1) / L;  // batches of a feature
        const uint64_t per = 16 * m * L                   // level buffer A
                             + 16 * ((m + 1) / 2) * 2 * L  // level buffer B
                             + 16 * 2 * bit_length(m) * L  // final merges
                             + 16 * L                       // compressed summary
                             + 8 * (m + 1)                  // entry counts
                             + sizeof(SkSortTask) * m + sizeof(SkMergeTask) * (m + bit_length(m)) +
                             sizeof(SkCutTask) + 4 * max_bin + 64;
        b += per * n_num;
    }
    return b;
}

uint64_t room_of(int device, uint64_t budget) {
    if (budget) return budget;
    size_t free_b = 0, total_b = 0;
    if (hipSetDevice(device) != hipSuccess || hipMemGetInfo(&free_b, &total_b) != hipSuccess)
        return 0;
    const uint64_t reserve = std::max<uint64_t>(free_b / 100 * 15, 512ull << 20);
    return free_b > reserve ? free_b - reserve : 0;
}

// gfx950 has 160 KiB of LDS per workgroup: opt a kernel in beyond the 64 KiB
// default (what its static LDS leaves).
template <class K>
hipError_t allow_lds(K kernel) {
    const void *fn = reinterpret_cast<const void *>(kernel);
    hipFuncAttributes fa{};
    hipError_t e = hipFuncGetAttributes(&fa, fn);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)(160 * 1024 - fa.sharedSizeBytes));
}

}  // namespace

struct fbh_sketch {
    int device = 0;
    hipStream_t stream = nullptr;
    uint64_t n_rows = 0, pushed = 0, stage_rows = 0;
    uint32_t nf = 0, max_bin = 0, n_num = 0;
    std::vector<uint8_t> cat;
    std::vector<int32_t> num_of;  // numeric index of a feature, -1 for categorical
    std::vector<void *> allocs;
    float *stage = nullptr, *comp = nullptr;
    uint32_t *cnt = nullptr, *off = nullptr, *zero = nullptr, *cat_bad = nullptr;
    int32_t *d_num_of = nullptr, *cat_max = nullptr;
    uint64_t *n_valid = nullptr;
    bool finished = false;

    template <class T>
    T *alloc(uint64_t count, const char *what) {
        void *p = nullptr;
        sk_check(hipMalloc(&p, std::max<uint64_t>(count * sizeof(T), 64)), what);
        allocs.push_back(p);
        return static_cast<T *>(p);
    }
    ~fbh_sketch() {
        if (stream) (void)hipStreamSynchronize(stream);
        for (void *p : allocs) (void)hipFree(p);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

uint32_t count_numeric(uint32_t nf, const uint8_t *cat) {
    uint32_t n = 0;
    for (uint32_t f = 0; f < nf; f++) n += (cat && cat[f]) ? 0u : 1u;
    return n;
}

}  // namespace

extern "C" {

uint64_t fbh_sketch_device_bytes(uint64_t n_rows, uint32_t n_features, uint32_t max_bin,
                                 const uint8_t *categorical) {
    if (max_bin > SK_MAX_BIN || n_rows >= (1ull << 32)) return 0;
    return sketch_bytes(n_rows, n_features, count_numeric(n_features, categorical), max_bin);
}

int fbh_sketch_fits(int device, uint64_t n_rows, uint32_t n_features, uint32_t max_bin,
                    const uint8_t *categorical, uint64_t memory_budget) {
    const uint64_t need = fbh_sketch_device_bytes(n_rows, n_features, max_bin, categorical);
    if (!need || !fbh_device_available(device)) return 0;
    return need <= room_of(device, memory_budget) ? 1 : 0;
}

int fbh_sketch_create(int device, uint64_t n_rows, uint32_t n_features, uint32_t max_bin,
                      const uint8_t *categorical, uint64_t memory_budget, fbh_sketch **out) {
    return sk_guard([&] {
        if (!out) throw SkError(FBH_INPUT_ERROR, "null argument");
        *out = nullptr;
        if (max_bin > SK_MAX_BIN)
            throw SkError(FBH_INPUT_ERROR, "the device sketch takes max_bin up to " +
                                               std::to_string(SK_MAX_BIN));
        if (n_rows >= (1ull << 32))
            throw SkError(FBH_INPUT_ERROR, "the device sketch takes fewer than 2^32 rows");
        if (!fbh_device_available(device))
            throw SkError(FBH_RUNTIME_ERROR, "device " + std::to_string(device) +
                                                 " is not an available gfx950 GPU");
        const uint64_t need = fbh_sketch_device_bytes(n_rows, n_features, max_bin, categorical);
        const uint64_t room = room_of(device, memory_budget);
        if (need > room)
            throw SkError(FBH_INPUT_ERROR, "the device sketch needs " + std::to_string(need) +
                                               " bytes, more than the " + std::to_string(room) +
                                               " bytes of room");
        std::unique_ptr<fbh_sketch> s(new fbh_sketch());
        s->device = device;
        s->n_rows = n_rows;
        s->nf = n_features;
        s->max_bin = max_bin;
        s->cat.assign(n_features, 0);
        s->num_of.assign(n_features, -1);
        for (uint32_t f = 0; f < n_features; f++) {
            s->cat[f] = categorical && categorical[f] ? 1 : 0;
            if (!s->cat[f]) s->num_of[f] = (int32_t)s->n_num++;
        }
        sk_check(hipSetDevice(device), "hipSetDevice");
        sk_check(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "stream creation");
        s->stage_rows = stage_rows_of(n_rows, n_features);
        const uint64_t tiles = (s->stage_rows + SK_ROWS - 1) / SK_ROWS;
        s->stage = s->alloc<float>(s->stage_rows * n_features, "sketch row staging");
        s->cnt = s->alloc<uint32_t>(tiles * s->n_num, "sketch counts");
        s->off = s->alloc<uint32_t>(tiles * s->n_num, "sketch offsets");
        s->comp = s->alloc<float>(n_rows * s->n_num, "sketch values");
        s->n_valid = s->alloc<uint64_t>(s->n_num, "sketch value counts");
        s->zero = s->alloc<uint32_t>(s->n_num, "sketch zero signs");
        s->cat_max = s->alloc<int32_t>(n_features, "sketch category codes");
        s->cat_bad = s->alloc<uint32_t>(n_features, "sketch category checks");
        s->d_num_of = s->alloc<int32_t>(n_features, "sketch feature map");
        sk_check(hipMemsetAsync(s->n_valid, 0, 8ull * std::max(s->n_num, 1u), s->stream), "memset");
        sk_check(hipMemsetAsync(s->zero, 0, 4ull * std::max(s->n_num, 1u), s->stream), "memset");
        sk_check(hipMemsetAsync(s->cat_max, 0xFF, 4ull * std::max(n_features, 1u), s->stream),
                 "memset");
        sk_check(hipMemsetAsync(s->cat_bad, 0, 4ull * std::max(n_features, 1u), s->stream), "memset");
        if (n_features)
            sk_check(hipMemcpyAsync(s->d_num_of, s->num_of.data(), 4ull * n_features,
                                    hipMemcpyHostToDevice, s->stream),
                     "feature map upload");
        sk_check(hipStreamSynchronize(s->stream), "sketch setup");
        *out = s.release();
    });
}

int fbh_sketch_push_rows(fbh_sketch *s, const float *x, uint64_t n_rows) {
    return sk_guard([&] {
        if (!s || (!x && n_rows)) throw SkError(FBH_INPUT_ERROR, "null argument");
        if (s->finished) throw SkError(FBH_INPUT_ERROR, "the sketch's cuts were already taken");
        if (n_rows > s->n_rows - s->pushed)
            throw SkError(FBH_INPUT_ERROR, "more rows pushed than the sketch was created for");
        if (n_rows == 0 || s->nf == 0) {
            s->pushed += n_rows;
            return;
        }
        sk_check(hipSetDevice(s->device), "hipSetDevice");
        const uint64_t nf = s->nf;
        for (uint64_t r = 0; r < n_rows; r += s->stage_rows) {
            const uint64_t b = std::min(s->stage_rows, n_rows - r);
            // Stream order: the copy waits for the previous chunk's kernels.
            sk_check(hipMemcpyAsync(s->stage, x + r * nf, 4 * b * nf, hipMemcpyHostToDevice,
                                    s->stream),
                     "row upload");
            const uint32_t tiles = (uint32_t)((b + SK_ROWS - 1) / SK_ROWS);
            const dim3 grid(tiles, (uint32_t)((nf + SK_FEATS - 1) / SK_FEATS));
            hipLaunchKernelGGL(sk_count_kernel, grid, dim3(SK_TPB), 0, s->stream, s->stage, b,
                               (uint32_t)nf, s->d_num_of, s->n_num, s->cnt, s->zero, s->cat_max,
                               s->cat_bad);
            sk_check(hipGetLastError(), "sketch count");
            if (s->n_num) {
                hipLaunchKernelGGL(sk_offsets_kernel, dim3(s->n_num), dim3(SK_TPB), 0, s->stream,
                                   s->cnt, tiles, s->n_num, s->off, s->n_valid);
                sk_check(hipGetLastError(), "sketch offsets");
                hipLaunchKernelGGL(sk_compact_kernel, grid, dim3(SK_TPB), 0, s->stream, s->stage, b,
                                   (uint32_t)nf, s->d_num_of, s->n_num, s->off, s->comp, s->n_rows);
                sk_check(hipGetLastError(), "sketch compaction");
            }
        }
        sk_check(hipStreamSynchronize(s->stream), "row sketching");  // the caller may reuse x
        s->pushed += n_rows;
    });
}

int fbh_sketch_missing(const fbh_sketch *s, uint64_t *missing) {
    return sk_guard([&] {
        if (!s || !missing) throw SkError(FBH_INPUT_ERROR, "null argument");
        sk_check(hipSetDevice(s->device), "hipSetDevice");
        std::vector<uint64_t> n_valid(s->n_num);
        if (s->n_num) {
            sk_check(hipMemcpyAsync(n_valid.data(), s->n_valid, 8ull * s->n_num,
                                    hipMemcpyDeviceToHost, s->stream),
                     "download");
            sk_check(hipStreamSynchronize(s->stream), "sync");
        }
        for (uint32_t f = 0; f < s->nf; f++)
            missing[f] = s->num_of[f] < 0 ? 0 : s->pushed - n_valid[(uint32_t)s->num_of[f]];
    });
}

int fbh_sketch_cuts(fbh_sketch *s, float *cut_values, uint64_t values_capacity,
                    uint32_t *cut_offsets, uint8_t *host_features) {
    return sk_guard([&] {
        if (!s || !cut_offsets || !host_features) throw SkError(FBH_INPUT_ERROR, "null argument");
        if (s->finished) throw SkError(FBH_INPUT_ERROR, "the sketch's cuts were already taken");
        s->finished = true;
        sk_check(hipSetDevice(s->device), "hipSetDevice");
        const uint32_t nf = s->nf, nn = s->n_num;
        std::vector<uint64_t> n_valid(nn);
        std::vector<uint32_t> zero(nn), cat_bad(nf);
        std::vector<int32_t> cat_max(nf);
        if (nn) {
            sk_check(hipMemcpyAsync(n_valid.data(), s->n_valid, 8ull * nn, hipMemcpyDeviceToHost,
                                    s->stream), "download");
            sk_check(hipMemcpyAsync(zero.data(), s->zero, 4ull * nn, hipMemcpyDeviceToHost,
                                    s->stream), "download");
        }
        if (nf) {
            sk_check(hipMemcpyAsync(cat_max.data(), s->cat_max, 4ull * nf, hipMemcpyDeviceToHost,
                                    s->stream), "download");
            sk_check(hipMemcpyAsync(cat_bad.data(), s->cat_bad, 4ull * nf, hipMemcpyDeviceToHost,
                                    s->stream), "download");
        }
        sk_check(hipStreamSynchronize(s->stream), "download");
        for (uint32_t f = 0; f < nf; f++)
            if (s->cat[f] && cat_bad[f])
                throw SkError(FBH_INPUT_ERROR,
                              "categorical feature #" + std::to_string(f) +
                                  " contains a value that is not an integer code in 0..=65533");

        // ---- the binary counter's layout ----
        const uint32_t max_bin = s->max_bin;
        const uint32_t n_cuts = max_bin >= 1 ? max_bin - 1 : 0;
        const uint64_t L = sk_limit(max_bin);
        std::vector<uint64_t> m(nn, 0), abase(nn + 1, 0), bbase(nn + 1, 0), tbase(nn + 1, 0);
        for (uint32_t j = 0; j < nn; j++) {
            m[j] = n_cuts ? (n_valid[j] + L - 1) / L : 0;
            abase[j + 1] = abase[j] + m[j];
            bbase[j + 1] = bbase[j] + (m[j] + 1) / 2;
            tbase[j + 1] = tbase[j] + (m[j] ? 2ull * __builtin_popcountll(m[j]) : 0ull);
        }
        std::vector<uint32_t> n_out(nn, 0);
        std::vector<float> cuts_dev;
        if (abase[nn]) {
            SkEntry *A = s->alloc<SkEntry>(abase[nn] * L, "sketch summaries");
            SkEntry *B = s->alloc<SkEntry>(bbase[nn] * 2 * L, "sketch summaries");
            SkEntry *Tm = s->alloc<SkEntry>(tbase[nn] * L, "sketch final merges");
            SkEntry *P = s->alloc<SkEntry>((uint64_t)nn * L, "sketch compressed summaries");
            uint32_t *cA = s->alloc<uint32_t>(abase[nn], "sketch entry counts");
            uint32_t *cB = s->alloc<uint32_t>(bbase[nn], "sketch entry counts");
            uint32_t *cT = s->alloc<uint32_t>(tbase[nn], "sketch entry counts");
            float *d_cuts = s->alloc<float>((uint64_t)nn * n_cuts, "sketch cuts");
            uint32_t *d_ncut = s->alloc<uint32_t>(nn, "sketch cut counts");
            // Level l's slot k of feature j: level 0 in A at limit entries a
            // slot, even levels above in A and odd levels in B at 2 limit
            // entries a slot. A block left alone at level l (an odd count of
            // them) sits in the last slot, beyond what level l + 2 writes.
            auto slot = [&](uint32_t l, uint32_t j, uint64_t k, const SkEntry **e, uint32_t **c) {
                if (l % 2 == 0) {
                    *e = A + abase[j] * L + k * (l == 0 ? L : 2 * L);
                    *c = cA + abase[j] + k;
                } else {
                    *e = B + bbase[j] * 2 * L + k * 2 * L;
                    *c = cB + bbase[j] + k;
                }
            };
            std::vector<SkSortTask> sorts;
            sorts.reserve(abase[nn]);
            for (uint32_t j = 0; j < nn; j++)
                for (uint64_t k = 0; k < m[j]; k++) {
                    const uint64_t len = std::min<uint64_t>(L, n_valid[j] - k * L);
                    sorts.push_back(SkSortTask{s->comp + (uint64_t)j * s->n_rows + k * L,
                                               A + (abase[j] + k) * L, cA + abase[j] + k,
                                               (uint32_t)len, 0});
                }
            std::vector<SkMergeTask> merges;
            std::vector<uint64_t> level_end;  // merges of levels 0..l end at level_end[l]
            for (uint32_t l = 0;; l++) {
                bool any = false;
                for (uint32_t j = 0; j < nn; j++) {
                    const uint64_t c = m[j] >> l;
                    for (uint64_t k = 0; k + 1 < c; k += 2) {
                        SkMergeTask t{};
                        const SkEntry *e;
                        uint32_t *cnt;
                        slot(l, j, k, &e, &cnt);
                        t.a = e;
                        t.na = cnt;
                        slot(l, j, k + 1, &e, &cnt);
                        t.b = e;
                        t.nb = cnt;
                        slot(l + 1, j, k / 2, &e, &cnt);
                        t.d = const_cast<SkEntry *>(e);
                        t.nd = cnt;
                        merges.push_back(t);
                        any = true;
                    }
                }
                if (!any) break;
                level_end.push_back(merges.size());
            }
            // collapse: the levels still held (the set bits of m), lowest first.
            std::vector<SkCutTask> cut_tasks;
            std::vector<std::vector<SkMergeTask>> finals;
            for (uint32_t j = 0; j < nn; j++) {
                if (!m[j]) continue;
                const SkEntry *cur = nullptr;
                uint32_t *cur_n = nullptr;
                uint32_t step = 0;
                uint64_t acc = 0;  // entries the merged result may hold, in limits
                for (uint32_t l = 0; (m[j] >> l) != 0; l++) {
                    if (!((m[j] >> l) & 1)) continue;
                    const SkEntry *e;
                    uint32_t *cnt;
                    slot(l, j, (m[j] >> l) - 1, &e, &cnt);
                    if (!cur) {
                        cur = e;
                        cur_n = cnt;
                        acc = 1;
                        continue;
                    }
                    acc++;
                    if (finals.size() <= step) finals.emplace_back();
                    SkMergeTask t{};
                    t.a = cur;
                    t.na = cur_n;
                    t.b = e;
                    t.nb = cnt;
                    const uint64_t half = tbase[j] + (step % 2) * (uint64_t)__builtin_popcountll(m[j]);
                    t.d = Tm + half * L;
                    t.nd = cT + tbase[j] + step;
                    finals[step].push_back(t);
                    cur = t.d;
                    cur_n = t.nd;
                    step++;
                }
                (void)acc;
                cut_tasks.push_back(SkCutTask{cur, cur_n, P + (uint64_t)j * L,
                                              d_cuts + (uint64_t)j * n_cuts, d_ncut + j, {0, 0}});
            }
            // One upload of every table.
            uint64_t n_final = 0;
            for (auto &f : finals) n_final += f.size();
            const uint64_t bytes = sizeof(SkSortTask) * sorts.size() +
                                   sizeof(SkMergeTask) * (merges.size() + n_final) +
                                   sizeof(SkCutTask) * cut_tasks.size();
            uint8_t *tab = s->alloc<uint8_t>(bytes, "sketch task tables");
            std::vector<uint8_t> host(bytes);
            uint64_t pos = 0;
            auto put = [&](const void *p, uint64_t nb) {
                if (nb) std::memcpy(host.data() + pos, p, nb);
                pos += nb;
            };
            const uint64_t o_sort = pos;
            put(sorts.data(), sizeof(SkSortTask) * sorts.size());
            const uint64_t o_merge = pos;
            put(merges.data(), sizeof(SkMergeTask) * merges.size());
            std::vector<uint64_t> o_final;
            for (auto &f : finals) {
                o_final.push_back(pos);
                put(f.data(), sizeof(SkMergeTask) * f.size());
            }
            const uint64_t o_cut = pos;
            put(cut_tasks.data(), sizeof(SkCutTask) * cut_tasks.size());
            sk_check(hipMemcpy(tab, host.data(), bytes, hipMemcpyHostToDevice), "task upload");

            // ---- launches ----
            const uint32_t Pk = pow2_at_least((uint32_t)L);
            sk_check(allow_lds(sk_sort_kernel), "LDS attribute");
            const uint32_t cut_lds = 4 * (uint32_t)L + 4 * max_bin;
            sk_check(allow_lds(sk_cuts_kernel), "LDS attribute");
            sk_check(allow_lds(sk_merge_kernel), "LDS attribute");
            hipLaunchKernelGGL(sk_sort_kernel, dim3((uint32_t)sorts.size()), dim3(SK_TPB),
                               4 * Pk, s->stream, reinterpret_cast<const SkSortTask *>(tab + o_sort),
                               Pk);
            sk_check(hipGetLastError(), "sketch batch summaries");
            uint64_t first = 0;
            for (uint64_t e : level_end) {
                hipLaunchKernelGGL(sk_merge_kernel, dim3((uint32_t)(e - first)), dim3(SK_TPB),
                                   2 * L, s->stream,
                                   reinterpret_cast<const SkMergeTask *>(tab + o_merge) + first,
                                   (uint32_t)L, 1u);
                sk_check(hipGetLastError(), "sketch merges");
                first = e;
            }
            for (size_t t = 0; t < finals.size(); t++) {
                hipLaunchKernelGGL(sk_merge_kernel, dim3((uint32_t)finals[t].size()), dim3(SK_TPB),
                                   0, s->stream,
                                   reinterpret_cast<const SkMergeTask *>(tab + o_final[t]),
                                   (uint32_t)L, 0u);
                sk_check(hipGetLastError(), "sketch final merges");
            }
            hipLaunchKernelGGL(sk_cuts_kernel, dim3((uint32_t)cut_tasks.size()), dim3(SK_TPB),
                               cut_lds, s->stream,
                               reinterpret_cast<const SkCutTask *>(tab + o_cut), (uint32_t)L,
                               max_bin);
            sk_check(hipGetLastError(), "sketch cuts");
            cuts_dev.resize((uint64_t)nn * n_cuts);
            sk_check(hipMemcpyAsync(n_out.data(), d_ncut, 4ull * nn, hipMemcpyDeviceToHost,
                                    s->stream), "download");
            sk_check(hipMemcpyAsync(cuts_dev.data(), d_cuts, 4ull * nn * n_cuts,
                                    hipMemcpyDeviceToHost, s->stream), "download");
            sk_check(hipStreamSynchronize(s->stream), "sketch");
        }

        // ---- the flat cuts ----
        uint64_t total = 0;
        for (uint32_t f = 0; f < nf; f++) {
            host_features[f] = 0;
            uint64_t c;
            if (s->cat[f]) {
                c = (uint64_t)std::max(cat_max[f], 0);
            } else {
                const uint32_t j = (uint32_t)s->num_of[f];
                c = m[j] ? n_out[j] : 0;
                if (zero[j] == 3u)
                    for (uint64_t i = 0; i < c; i++)
                        if (cuts_dev[(uint64_t)j * n_cuts + i] == 0.0f) host_features[f] = 1;
                if (host_features[f]) c = 0;
            }
            cut_offsets[f] = (uint32_t)total;
            total += c;
        }
        cut_offsets[nf] = (uint32_t)total;
        if (total > values_capacity)
            throw SkError(FBH_INPUT_ERROR, "cut_values holds " + std::to_string(values_capacity) +
                                               " values, the cuts need " + std::to_string(total));
        for (uint32_t f = 0; f < nf; f++) {
            float *o = cut_values + cut_offsets[f];
            const uint32_t c = cut_offsets[f + 1] - cut_offsets[f];
            if (s->cat[f]) {
                for (uint32_t i = 0; i < c; i++) o[i] = (float)(i + 1);
            } else if (c) {
                std::memcpy(o, cuts_dev.data() + (uint64_t)s->num_of[f] * n_cuts, 4ull * c);
            }
        }
    });
}

int fbh_sketch_destroy(fbh_sketch *s) {
    return sk_guard([&] { delete s; });
}

}  // extern "C"
