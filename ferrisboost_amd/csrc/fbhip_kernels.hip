// fbhip_kernels.hip -- CDNA4 (gfx950) kernels of the training and explanation
// backend. Built with -ffp-contract=off and correctly rounded f32 division so
// every floating-point step rounds exactly like the host engine.
//
// Kernels:
//   hist_kernel          fixed-point gradient histograms, LDS-privatised per
//                        tile, batched over the nodes of a level
//                        (reference: histogram.cu:1685-1852)
//   subtract_kernel      sibling subtraction (hist.rs:391-400)
//   split_feat_kernel    split-gain scan of one (node, feature)
//                        (split.rs:331-617, histogram.cu:250-510)
//   split_node_kernel    per-node argmax over features (split.rs:631-642)
//   part_*_kernel        stable row partition (mod.rs:5169-5430,
//                        histogram.cu:2029-2395)
//   leaf_kernel          leaf value scatter into the prediction delta
//                        (histogram.cu:2397-2441)
//   gpair_*_kernel       device quantisation (histogram.cu:1079-1177)
//   shap_kernel          QuadratureTreeSHAP (explain.rs:303-401, 704-728)

#include "fb_expf.h"
#include "fb_tanhf.h"
#include "fbhip_internal.h"
#include "fbhip_quant.h"

#include <hip/hip_ext.h>

#include <math.h>

#include <algorithm>
#include <type_traits>

namespace fbh {

// ======================================================================
// histogram
// ======================================================================

template <int RD>
__device__ __forceinline__ void load_record(const uint8_t *p, uint32_t (&r)[RD]) {
    if constexpr (RD % 4 == 0) {
#pragma unroll
        for (int q = 0; q < RD / 4; q++) {
            uint4 v = reinterpret_cast<const uint4 *>(p)[q];
            r[4 * q + 0] = v.x;
            r[4 * q + 1] = v.y;
            r[4 * q + 2] = v.z;
            r[4 * q + 3] = v.w;
        }
    } else if constexpr (RD % 2 == 0) {
#pragma unroll
        for (int q = 0; q < RD / 2; q++) {
            uint2 v = reinterpret_cast<const uint2 *>(p)[q];
            r[2 * q + 0] = v.x;
            r[2 * q + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int q = 0; q < RD; q++) r[q] = reinterpret_cast<const uint32_t *>(p)[q];
    }
}

// Workgroup -> (tile, chunk). XCD-local (few tiles): every tile of chunk c
// runs on XCD c % 8, so the chunk's row ids and pairs come from HBM once
// into that XCD's L2. Linear (many tiles, few chunks): consecutive
// workgroups take consecutive tiles of one chunk, spreading every chunk over
// all XCDs, so no XCD idles when there are fewer than 8 chunks.
__device__ __forceinline__ void block_to_work(const HistLaunch &L, uint32_t b, uint32_t &tile_i,
                                              uint32_t &chunk) {
    if (L.linear) {
        tile_i = b % L.n_tiles;
        chunk = b / L.n_tiles;
        return;
    }
    const uint32_t xcd = b % XCDS;
    const uint32_t k = b / XCDS;
    tile_i = k % L.n_tiles;
    chunk = (k / L.n_tiles) * XCDS + xcd;
}

__device__ __forceinline__ void lds_add_u64(unsigned long long *p, unsigned long long v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void global_add_u64(unsigned long long *p, unsigned long long v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One workgroup accumulates one chunk of one node's rows into the LDS
// histogram of one tile, then merges it into the node's histogram slot:
// a plain store when the node has a single chunk, 64-bit global atomics
// otherwise. Fixed-point addition is exact and order independent, so the
// result equals the host engine's bit for bit.
//
// Workgroup -> (chunk, tile) follows block_to_work.
//
// LDS layout is planar: slots [0, S) hold gradient sums, [S, 2S) Hessian
// sums (S = tile slots + 64). The last 64 slots of each plane are one dummy
// slot per lane: a missing / unseen / unselected cell adds zero there instead
// of branching, so the atomic stream has no divergent control flow.
// Interleaved tiles (ROT: 16 features of 8 bits in a 16-byte record, or of
// 16 bits with at most 256 bins each in a 32-byte record) use the
// interleaved layout instead: slot bin * 16 + k for feature k of the tile,
// the plane HIST_ROT_SLOTS + 64 slots long, and lane l takes the record's
// features in the order l, l + 1, ... (mod 16). The 64 lanes of one LDS atomic then hit
// 16 features, four lanes each, and slot bin * 16 + k sits in bank pair k
// whatever the bin: every bank pair takes exactly four lanes, where the
// planar layout's random bins pile up to twice that on one pair. The dummy
// of lane l for feature k is HIST_ROT_SLOTS + 16 * (l / 16) + k, in the same
// bank pair. Measured on an MI355X: 4.9 vs 2.8 T 64-bit LDS adds per second.
// STREAM: the tile is streamed; the launch covers the rows of one window
// [L.row_lo, L.row_hi), whose records are at L.stream_data, and every node's
// histogram accumulates over several launches (global atomics only).
template <int W, int RD, int UNROLL, int TPB, bool STREAM, bool ROT>
__global__ __launch_bounds__(TPB) void hist_kernel(const HistLaunch L) {
    extern __shared__ unsigned long long lds[];
    constexpr int FPD = 4 / W;
    constexpr int NF = RD * FPD;
    constexpr uint32_t MASK = W == 1 ? 0xFFu : 0xFFFFu;
    static_assert(!ROT || NF == 16, "interleaved layout: 16 features a record");
    static_assert(TPB % 64 == 0, "whole waves");

    uint32_t tile_i, chunk;
    block_to_work(L, blockIdx.x, tile_i, chunk);
    if (chunk >= L.n_chunks) return;
    const TileDev T = L.tiles[tile_i];
    const uint32_t n_nodes = L.dev_n_nodes ? *L.dev_n_nodes : L.n_nodes;
    if (n_nodes == 0) return;

    uint32_t lo = 0, hi = n_nodes;
    while (hi - lo > 1) {
        uint32_t mid = (lo + hi) >> 1;
        if (L.nodes[mid].chunk_begin <= chunk) lo = mid;
        else hi = mid;
    }
    const HistNodeDev N = L.nodes[lo];
    // A device-planned grid is an upper bound: chunks past the last node's
    // end have no rows.
    if (chunk - N.chunk_begin >= N.n_chunks) return;
    const uint32_t chunk_rows = L.dev_chunk_rows ? *L.dev_chunk_rows : L.chunk_rows;
    uint32_t r0 = (chunk - N.chunk_begin) * chunk_rows;
    uint32_t r1 = min(r0 + chunk_rows, N.row_len);
    if (STREAM) {
        // A node's row ids ascend (stable partitions of 0..n), so the rows of
        // the window are one sub-range of the chunk: two lower bounds.
        __shared__ uint32_t win[2];
        if (threadIdx.x < 2) {
            const uint32_t key = threadIdx.x == 0 ? L.row_lo : L.row_hi;
            const uint32_t *rr = L.rows + N.row_off;
            uint32_t a = r0, b = r1;
            while (a < b) {
                const uint32_t m = (a + b) >> 1;
                if (rr[m] < key) a = m + 1;
                else b = m;
            }
            win[threadIdx.x] = a;
        }
        __syncthreads();
        r0 = win[0];
        r1 = win[1];
        if (r0 >= r1) return;  // uniform: no row of this chunk in the window
    }

    const uint32_t tid = threadIdx.x;
    // Interleaved layout: the lane's rotation and, per step k, the bin count
    // of its feature (k + rot) mod 16. Planar: per feature.
    const uint32_t rot = tid & 15u;
    uint32_t nb[NF], loff[NF];
    uint32_t hot0[ROT ? 1 : NF], hot1[ROT ? 1 : NF], hoff[ROT ? 1 : NF];
#pragma unroll
    for (int k = 0; k < NF; k++) {
        const uint32_t fi = ROT ? ((uint32_t)k + rot) & 15u : (uint32_t)k;
        if (fi < T.n_feat) {
            const TileFeatDev F = L.feats[T.feat_base + fi];
            nb[k] = F.n_bins;
            loff[k] = F.lds_off;
            if constexpr (!ROT) {
                hot0[k] = F.hot[0];
                hot1[k] = F.hot[1];
                hoff[k] = F.hot_off + (tid & 63u);
            }
        } else {
            nb[k] = 0;
            loff[k] = 0;
            if constexpr (!ROT) {
                hot0[k] = hot1[k] = HOT_NONE;
                hoff[k] = 0;
            }
        }
    }

    // plane size incl. the per-lane dummies
    const uint32_t S = ROT ? HIST_ROT_SLOTS + 64u : T.lds_slots + 64u;
    for (uint32_t i = tid; i < 2 * S; i += TPB) lds[i] = 0ull;
    __syncthreads();
    const uint32_t dummy = ROT ? HIST_ROT_SLOTS + 16u * ((tid & 63u) >> 4) : T.lds_slots + (tid & 63u);
    unsigned long long *gplane = lds;
    unsigned long long *hplane = lds + S;

    // A null row arena: the node's rows are row_off, row_off + 1, ... (the
    // root before any partition).
    const uint32_t *rows = L.rows ? L.rows + N.row_off : nullptr;
    const longlong2 *gp = reinterpret_cast<const longlong2 *>(L.gpair);
    // f32 pairs: quantized by shifts (the scales are powers of two).
    const float2 *gf = reinterpret_cast<const float2 *>(L.gpair_f32);
    int lg = 0, lh = 0;
    if (gf) {
        lg = pow2_exponent(L.scales->scale[0]);
        lh = pow2_exponent(L.scales->scale[1]);
    }
    // Interleaved layout: the gradient plane plus 8 bytes per slot of the
    // feature the lane takes at step k, (k + rot) mod 16.
    char *fptr[NF];
#pragma unroll
    for (int k = 0; k < NF; k++)
        fptr[k] = reinterpret_cast<char *>(gplane) + ((((uint32_t)k + rot) & 15u) << 3);
    // The row loop, compiled once per pair format (no per-row branch).
    auto accumulate = [&](auto pair_f32) {
        constexpr bool PF = decltype(pair_f32)::value;
        for (uint32_t i = r0 + tid; i < r1; i += TPB * UNROLL) {
            uint32_t row[UNROLL];
            bool ok[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; u++) {
                const uint32_t idx = i + u * TPB;
                ok[u] = idx < r1;
                row[u] = ok[u] ? (rows ? rows[idx] : N.row_off + idx) : 0u;
            }
            longlong2 g[UNROLL];
            float2 f[UNROLL];
            uint32_t rec[UNROLL][RD];
#pragma unroll
            for (int u = 0; u < UNROLL; u++) {
                if (ok[u]) {
                    if constexpr (PF) f[u] = gf[row[u]];
                    else g[u] = gp[row[u]];
                    const uint8_t *src = STREAM ? L.stream_data + (size_t)(row[u] - L.row_lo) * T.stride
                                                : T.data + (size_t)row[u] * T.stride;
                    if (ROT || T.rec_dwords == RD) {
                        load_record<RD>(src, rec[u]);
                    } else {
                        // A smaller record than the launch's (planar tiles of
                        // one width share a launch): its dwords only.
#pragma unroll
                        for (int d = 0; d < RD; d++)
                            rec[u][d] = d < (int)T.rec_dwords
                                            ? reinterpret_cast<const uint32_t *>(src)[d]
                                            : 0u;
                    }
                } else {
                    f[u] = make_float2(0.0f, 0.0f);
                    g[u] = make_longlong2(0, 0);
#pragma unroll
                    for (int d = 0; d < RD; d++) rec[u][d] = 0u;
                }
            }
            if constexpr (PF) {
#pragma unroll
                for (int u = 0; u < UNROLL; u++)
                    g[u] = make_longlong2(quantize_pow2(f[u].x, lg), quantize_pow2(f[u].y, lh));
            }
            if constexpr (ROT) {
                // Rotate each record right by rot features: cell k becomes the
                // cell of feature (k + rot) mod 16. Whole dwords first (a
                // barrel shifter over the record's RD dwords), then the
                // remaining cells within a dword (bytes).
                const uint32_t dsh = rot / FPD, bsh = (rot % FPD) * W;
#pragma unroll
                for (int u = 0; u < UNROLL; u++) {
                    uint32_t a[RD];
#pragma unroll
                    for (int j = 0; j < RD; j++) a[j] = rec[u][j];
#pragma unroll
                    for (int st = 1; st < RD; st <<= 1) {
                        uint32_t b[RD];
#pragma unroll
                        for (int j = 0; j < RD; j++) b[j] = (dsh & (uint32_t)st) ? a[(j + st) % RD] : a[j];
#pragma unroll
                        for (int j = 0; j < RD; j++) a[j] = b[j];
                    }
#pragma unroll
                    for (int j = 0; j < RD; j++)
                        rec[u][j] = __builtin_amdgcn_alignbyte(a[(j + 1) % RD], a[j], bsh);
                }
            }
#pragma unroll
            for (int u = 0; u < UNROLL; u++) {
                const unsigned long long gg = (unsigned long long)g[u].x;
                const unsigned long long hh = (unsigned long long)g[u].y;
#pragma unroll
                for (int d = 0; d < RD; d++) {
#pragma unroll
                    for (int q = 0; q < FPD; q++) {
                        const int fi = d * FPD + q;
                        const uint32_t bin = (rec[u][d] >> (q * 8 * W)) & MASK;
                        uint32_t s;
                        if (ROT) {
                            // Features outside the tile or not built this tree
                            // have nb 0 and add into the lane's dummy. Slot
                            // bin * 16 + feat (or the dummy's) in bytes, from
                            // the step's feature pointer.
                            unsigned long long *p = reinterpret_cast<unsigned long long *>(
                                fptr[fi] + (bin < nb[fi] ? bin << 7 : dummy << 3));
                            lds_add_u64(p, gg);
                            lds_add_u64(p + S, hh);
                            continue;
                        } else {
                            if (fi >= (int)T.n_feat) continue;  // uniform
                            if (nb[fi] == 0) continue;  // not built this tree (uniform)
                            // Missing (all ones) and unseen-category codes are >= n_bins;
                            // out-of-range rows (ok false) carry a zero pair. A hot
                            // bin goes to the lane's own slot of that bin.
                            s = bin < nb[fi] ? loff[fi] + bin : dummy;
                            if constexpr (!ROT) {
                                s = bin == hot0[fi] ? hoff[fi] : s;
                                s = bin == hot1[fi] ? hoff[fi] + 64u : s;
                            }
                        }
                        lds_add_u64(gplane + s, gg);
                        lds_add_u64(hplane + s, hh);
                    }
                }
            }
        }
    };
    if (gf) accumulate(std::true_type{});
    else accumulate(std::false_type{});
    __syncthreads();

    // One chunk: its slot. Several: the chunk's partial histogram, or
    // atomics into the cleared slot.
    const bool single = !STREAM && N.n_chunks == 1;
    const bool partial = !STREAM && !single && L.partials;
    int64_t *out = partial ? L.partials + (uint64_t)chunk * L.hist_width * 2u
                           : L.hist + (uint64_t)N.slot * L.hist_width * 2u;
    // A node of more than REDUCE_GROUP chunks is summed into its slot by
    // atomics (reduce_chunks_kernel): its first chunk's workgroups clear the
    // slot's bins of their tile here, so nothing clears it before.
    unsigned long long *clr =
        (partial && chunk == N.chunk_begin && N.n_chunks > L.clear_above)
            ? reinterpret_cast<unsigned long long *>(L.hist + (uint64_t)N.slot * L.hist_width * 2u)
            : nullptr;
    if (ROT) {
        // Slots in order (conflict-free LDS reads): each thread keeps one
        // feature, tid mod 16, and a wave writes 4 bins of 16 features.
        TileFeatDev F{};
        if (rot < T.n_feat) F = L.feats[T.feat_base + rot];
        for (uint32_t j = tid; j < HIST_ROT_SLOTS; j += TPB) {
            const uint32_t bin = j >> 4;
            if (bin >= F.n_bins) continue;
            const unsigned long long gg = gplane[j];
            const unsigned long long hh = hplane[j];
            unsigned long long *dst =
                reinterpret_cast<unsigned long long *>(out + 2u * (F.hist_off + bin));
            if (single || partial) {
                dst[0] = gg;
                dst[1] = hh;
            } else if ((gg | hh) != 0ull) {
                global_add_u64(dst, gg);
                global_add_u64(dst + 1, hh);
            }
            if (clr) {
                clr[2u * (F.hist_off + bin)] = 0ull;
                clr[2u * (F.hist_off + bin) + 1u] = 0ull;
            }
        }
        return;
    }
    for (uint32_t fi = 0; fi < T.n_feat; fi++) {
        const TileFeatDev F = L.feats[T.feat_base + fi];
        for (uint32_t bin = tid; bin < F.n_bins; bin += TPB) {
            unsigned long long gg = gplane[F.lds_off + bin];
            unsigned long long hh = hplane[F.lds_off + bin];
            // a hot bin: its 64 lane slots (integer sums, any order)
            const int hk = bin == F.hot[0] ? 0 : bin == F.hot[1] ? 1 : -1;
            if (hk >= 0) {
                const uint32_t b = F.hot_off + 64u * (uint32_t)hk;
                for (uint32_t l = 0; l < 64; l++) {
                    gg += gplane[b + l];
                    hh += hplane[b + l];
                }
            }
            unsigned long long *dst =
                reinterpret_cast<unsigned long long *>(out + 2u * (F.hist_off + bin));
            if (single || partial) {
                dst[0] = gg;
                dst[1] = hh;
            } else if ((gg | hh) != 0ull) {
                global_add_u64(dst, gg);
                global_add_u64(dst + 1, hh);
            }
            if (clr) {
                clr[2u * (F.hist_off + bin)] = 0ull;
                clr[2u * (F.hist_off + bin) + 1u] = 0ull;
            }
        }
    }
}

// A feature whose histogram does not fit an LDS tile (wide 16-bit bins)
// accumulates straight into the node's zeroed histogram with 64-bit global
// atomics; each tile of this kind holds one feature.
template <int W>
__global__ __launch_bounds__(HIST_TPB) void hist_global_kernel(const HistLaunch L) {
    uint32_t tile_i, chunk;
    block_to_work(L, blockIdx.x, tile_i, chunk);
    if (chunk >= L.n_chunks) return;
    const TileDev T = L.tiles[tile_i];
    const TileFeatDev F = L.feats[T.feat_base];
    if (F.n_bins == 0) return;
    const uint32_t n_nodes = L.dev_n_nodes ? *L.dev_n_nodes : L.n_nodes;
    if (n_nodes == 0) return;
    uint32_t lo = 0, hi = n_nodes;
    while (hi - lo > 1) {
        uint32_t mid = (lo + hi) >> 1;
        if (L.nodes[mid].chunk_begin <= chunk) lo = mid;
        else hi = mid;
    }
    const HistNodeDev N = L.nodes[lo];
    if (chunk - N.chunk_begin >= N.n_chunks) return;
    const uint32_t chunk_rows = L.dev_chunk_rows ? *L.dev_chunk_rows : L.chunk_rows;
    const uint32_t r0 = (chunk - N.chunk_begin) * chunk_rows;
    const uint32_t r1 = min(r0 + chunk_rows, N.row_len);
    unsigned long long *out = reinterpret_cast<unsigned long long *>(
        L.hist + ((uint64_t)N.slot * L.hist_width + F.hist_off) * 2u);
    const uint32_t *rows = L.rows ? L.rows + N.row_off : nullptr;
    const longlong2 *gp = reinterpret_cast<const longlong2 *>(L.gpair);
    const float2 *gf = reinterpret_cast<const float2 *>(L.gpair_f32);
    int lg = 0, lh = 0;
    if (gf) {
        lg = pow2_exponent(L.scales->scale[0]);
        lh = pow2_exponent(L.scales->scale[1]);
    }
    for (uint32_t i = r0 + threadIdx.x; i < r1; i += HIST_TPB) {
        const uint32_t row = rows ? rows[i] : N.row_off + i;
        longlong2 g;
        if (gf) {
            const float2 v = gf[row];
            g = make_longlong2(quantize_pow2(v.x, lg), quantize_pow2(v.y, lh));
        } else {
            g = gp[row];
        }
        if ((g.x | g.y) == 0) continue;
        const uint8_t *p = T.data + (size_t)row * T.stride;
        const uint32_t bin = W == 1 ? (uint32_t)p[0] : (uint32_t)*reinterpret_cast<const uint16_t *>(p);
        if (bin < F.n_bins) {
            global_add_u64(out + 2u * bin, (unsigned long long)g.x);
            global_add_u64(out + 2u * bin + 1, (unsigned long long)g.y);
        }
    }
}

hipError_t launch_hist_global(const HistLaunch &L, int width, hipEvent_t ev_start,
                              hipEvent_t ev_stop, hipStream_t s) {
    const uint32_t blocks = L.linear ? L.n_chunks * L.n_tiles : L.chunk_groups * XCDS * L.n_tiles;
    if (blocks == 0) return hipSuccess;
    if (width == 1)
        hipExtLaunchKernelGGL(hist_global_kernel<1>, dim3(blocks), dim3(HIST_TPB), 0, s, ev_start,
                              ev_stop, 0, L);
    else
        hipExtLaunchKernelGGL(hist_global_kernel<2>, dim3(blocks), dim3(HIST_TPB), 0, s, ev_start,
                              ev_stop, 0, L);
    return hipGetLastError();
}

template <int W, int RD, int TPB, bool STREAM, bool ROT>
static hipError_t launch_hist_t(const HistLaunch &L, size_t lds, hipEvent_t ev_start,
                                hipEvent_t ev_stop, hipStream_t s) {
    const uint32_t blocks = L.linear ? L.n_chunks * L.n_tiles : L.chunk_groups * XCDS * L.n_tiles;
    if (blocks == 0) return hipSuccess;
    // gfx950 has 160 KiB of LDS per workgroup; opt in beyond the 64 KiB
    // default (a per-function attribute, set once per device).
    static uint64_t attr_done = 0;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 64 && !(attr_done >> dev & 1)) {
        // The dynamic share is what the kernel's static LDS leaves of 160 KiB.
        const void *fn = reinterpret_cast<const void *>(&hist_kernel<W, RD, 4, TPB, STREAM, ROT>);
        hipFuncAttributes fa{};
        e = hipFuncGetAttributes(&fa, fn);
        if (e != hipSuccess) return e;
        e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(160 * 1024 - fa.sharedSizeBytes));
        if (e != hipSuccess) return e;
        attr_done |= 1ull << dev;
    }
    // Timing events ride on the dispatch itself (no separate marker packets).
    hipExtLaunchKernelGGL((hist_kernel<W, RD, 4, TPB, STREAM, ROT>), dim3(blocks), dim3(TPB),
                          (uint32_t)lds, s, ev_start, ev_stop, 0, L);
    return hipGetLastError();
}

template <int W, int RD, bool ROT>
static hipError_t launch_hist_wr(const HistLaunch &L, int tpb, bool stream, size_t lds,
                                 hipEvent_t e0, hipEvent_t e1, hipStream_t s) {
    if (stream) return launch_hist_t<W, RD, 256, true, ROT>(L, lds, e0, e1, s);
    if (tpb == 256) return launch_hist_t<W, RD, 256, false, ROT>(L, lds, e0, e1, s);
    if (tpb == 512) return launch_hist_t<W, RD, 512, false, ROT>(L, lds, e0, e1, s);
    if (tpb == 1024) return launch_hist_t<W, RD, 1024, false, ROT>(L, lds, e0, e1, s);
    return hipErrorInvalidValue;
}

hipError_t launch_hist(const HistLaunch &L, int width, int rd, bool rot, int tpb, bool stream,
                       size_t lds, hipEvent_t ev_start, hipEvent_t ev_stop, hipStream_t s) {
#define FBH_HIST_WR(WW, R, RT) \
    if (width == WW && rd == R && rot == RT) \
        return launch_hist_wr<WW, R, RT>(L, tpb, stream, lds, ev_start, ev_stop, s);
    FBH_HIST_WR(1, 1, false) FBH_HIST_WR(1, 2, false) FBH_HIST_WR(1, 3, false)
    FBH_HIST_WR(1, 4, true) FBH_HIST_WR(1, 8, false) FBH_HIST_WR(1, 12, false)
    FBH_HIST_WR(1, 16, false)
    FBH_HIST_WR(2, 1, false) FBH_HIST_WR(2, 2, false) FBH_HIST_WR(2, 3, false)
    FBH_HIST_WR(2, 4, false) FBH_HIST_WR(2, 8, false) FBH_HIST_WR(2, 8, true)
    FBH_HIST_WR(2, 12, false) FBH_HIST_WR(2, 16, false)
#undef FBH_HIST_WR
    return hipErrorInvalidValue;
}

// Zero whole histogram slots before atomic accumulation.
__global__ void zero_slots_kernel(int64_t *hist, uint64_t width, const uint32_t *slots) {
    int64_t *base = hist + (uint64_t)slots[blockIdx.y] * width * 2u;
    const uint64_t n = width * 2u;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        base[i] = 0;
}

hipError_t launch_zero_slots(int64_t *hist, uint64_t width, const uint32_t *slots, uint32_t n,
                             hipStream_t s) {
    if (n == 0) return hipSuccess;
    uint32_t bx = (uint32_t)std::min<uint64_t>((width * 2 + 255) / 256, 1024);
    hipLaunchKernelGGL(zero_slots_kernel, dim3(bx, n), dim3(256), 0, s, hist, width, slots);
    return hipGetLastError();
}

// Grid (word blocks, groups; a workgroup takes groups blockIdx.y + k *
// gridDim.y): group y belongs to the node whose group_begin range holds it.
// A node of at most REDUCE_GROUP chunks has one
// group, which sums them and stores the slot (zeros for a node without rows);
// a larger node's groups each add the sum of their REDUCE_GROUP chunks into
// its slot, which the histogram launch cleared (its first chunk's
// workgroups).
__global__ __launch_bounds__(256) void reduce_chunks_kernel(int64_t *hist, uint64_t width,
                                                           const int64_t *partials,
                                     const HistNodeDev *nodes, uint32_t n_nodes,
                                     const uint32_t *dev_n, uint32_t max_groups,
                                     uint32_t min_chunks) {
    // The node count and, speculatively (up to the host's bound, which the
    // node table holds), the nodes are requested together; the nodes then
    // come from LDS when they fit.
    constexpr uint32_t LDS_NODES = 256;  // the block size
    __shared__ uint4 s_nodes[LDS_NODES];  // chunk_begin, slot, n_chunks, group_begin
    const uint32_t bound = min(n_nodes, LDS_NODES);
    uint4 mine = make_uint4(0u, 0u, 0u, 0u);
    if (threadIdx.x < bound)
        mine = make_uint4(nodes[threadIdx.x].chunk_begin, nodes[threadIdx.x].slot,
                          nodes[threadIdx.x].n_chunks, nodes[threadIdx.x].group_begin);
    const uint32_t n = dev_n ? *dev_n : n_nodes;
    if (n == 0) return;
    const bool in_lds = n <= LDS_NODES;
    if (in_lds) {
        if (threadIdx.x < n) s_nodes[threadIdx.x] = mine;
        __syncthreads();
    }
    auto node_at = [&](uint32_t i) -> uint4 {
        return in_lds ? s_nodes[i]
                      : make_uint4(nodes[i].chunk_begin, nodes[i].slot, nodes[i].n_chunks,
                                   nodes[i].group_begin);
    };
    // Groups past the last node's (max_groups is an upper bound) are skipped.
    const uint4 last = node_at(n - 1);
    const uint32_t n_groups = min(max_groups, last.w + reduce_groups(last.z));
    if (blockIdx.y >= n_groups) return;
    const uint64_t W = width * 2u;
    const unsigned long long *src = reinterpret_cast<const unsigned long long *>(partials);
    for (uint32_t y = blockIdx.y; y < n_groups; y += gridDim.y) {
        uint32_t lo = 0, hi = n;
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) >> 1;
            if ((in_lds ? s_nodes[mid].w : nodes[mid].group_begin) <= y) lo = mid;
            else hi = mid;
        }
        const uint4 N = node_at(lo);  // chunk_begin, slot, n_chunks, group_begin
        const uint32_t g = y - N.w;
        // past the groups / written / left to split_pair_kernel
        if (g >= reduce_groups(N.z) || N.z == 1 || N.z < min_chunks) continue;
        const uint32_t c0 = g * REDUCE_GROUP, c1 = min(c0 + REDUCE_GROUP, N.z);
        const bool store = N.z <= REDUCE_GROUP;
        unsigned long long *dst = reinterpret_cast<unsigned long long *>(hist + (uint64_t)N.y * W);
        const unsigned long long *base = src + (uint64_t)(N.x + c0) * W;
        for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < W;
             i += (uint64_t)gridDim.x * blockDim.x) {
            // Four chunks' loads in flight at a time (a chunk past the
            // group's reads its first chunk again and adds nothing).
            unsigned long long sum = 0;
            for (uint32_t k = 0; k < c1 - c0; k += 4) {
                unsigned long long v[4];
#pragma unroll
                for (uint32_t q = 0; q < 4; q++)
                    v[q] = base[(uint64_t)(k + q < c1 - c0 ? k + q : 0u) * W + i];
#pragma unroll
                for (uint32_t q = 0; q < 4; q++) sum += k + q < c1 - c0 ? v[q] : 0ull;
            }
            if (store) dst[i] = sum;
            else if (sum) global_add_u64(dst + i, sum);
        }
    }
}

hipError_t launch_reduce_chunks(int64_t *hist, uint64_t width, const int64_t *partials,
                                const HistNodeDev *nodes, uint32_t n, const uint32_t *dev_n,
                                uint32_t max_groups, uint32_t min_chunks, hipStream_t s) {
    if (n == 0 || max_groups == 0) return hipSuccess;
    const uint32_t bx = (uint32_t)std::min<uint64_t>((width * 2 + 255) / 256, 1024);
    // About 16384 workgroups: a launch whose groups are mostly empty (their
    // nodes are summed elsewhere, or the bound is loose) costs little to
    // dispatch; the workgroups of a wide histogram loop over the groups.
    const uint32_t gy = std::min<uint32_t>(max_groups, std::max<uint32_t>(1, 16384 / bx));
    hipLaunchKernelGGL(reduce_chunks_kernel, dim3(bx, gy), dim3(256), 0, s, hist, width,
                       partials, nodes, n, dev_n, max_groups, min_chunks);
    return hipGetLastError();
}

// dst = parent - sibling, elementwise wrapping i64 (triples: dst, parent, sibling).
__global__ void subtract_kernel(int64_t *hist, uint64_t width, const uint32_t *triples,
                                const uint32_t *dev_n) {
    if (dev_n && blockIdx.y >= *dev_n) return;
    const uint32_t *t = triples + 3u * blockIdx.y;
    uint64_t *dst = reinterpret_cast<uint64_t *>(hist + (uint64_t)t[0] * width * 2u);
    const uint64_t *par = reinterpret_cast<const uint64_t *>(hist + (uint64_t)t[1] * width * 2u);
    const uint64_t *sib = reinterpret_cast<const uint64_t *>(hist + (uint64_t)t[2] * width * 2u);
    const uint64_t n = width * 2u;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = par[i] - sib[i];
}

hipError_t launch_subtract(int64_t *hist, uint64_t width, const uint32_t *triples, uint32_t n,
                           const uint32_t *dev_n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    uint32_t bx = (uint32_t)std::min<uint64_t>((width * 2 + 255) / 256, 1024);
    hipLaunchKernelGGL(subtract_kernel, dim3(bx, n), dim3(256), 0, s, hist, width, triples, dev_n);
    return hipGetLastError();
}

// group nonzero: per-chunk partials; only nodes of more chunks than that
// accumulate atomically. Otherwise every node of several (or no) chunks.
__global__ void zero_nodes_kernel(int64_t *hist, uint64_t width, const HistNodeDev *nodes,
                                  const uint32_t *dev_n, bool force, uint32_t group) {
    if (dev_n && blockIdx.y >= *dev_n) return;
    const HistNodeDev N = nodes[blockIdx.y];
    const bool clear = group ? N.n_chunks > group : (force || N.n_chunks != 1);
    if (!clear) return;  // written by plain stores
    int64_t *base = hist + (uint64_t)N.slot * width * 2u;
    const uint64_t n = width * 2u;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        base[i] = 0;
}

hipError_t launch_zero_nodes(int64_t *hist, uint64_t width, const HistNodeDev *nodes, uint32_t n,
                             const uint32_t *dev_n, bool force, uint32_t group, hipStream_t s) {
    if (n == 0) return hipSuccess;
    uint32_t bx = (uint32_t)std::min<uint64_t>((width * 2 + 255) / 256, 1024);
    hipLaunchKernelGGL(zero_nodes_kernel, dim3(bx, n), dim3(256), 0, s, hist, width, nodes, dev_n,
                       force, group);
    return hipGetLastError();
}

// Exclusive scan of v over the 1024 threads of the block (carry added by the
// caller); returns this thread's prefix and sets total.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t t = __shfl_up(v, off, 64);
        if (lane >= (uint32_t)off) v += t;
    }
    return v;
}

// Exclusive block scan: wave scans by shuffles, then one wave scans the
// wave totals (blockDim.x a multiple of 64, at most 1024; buf needs 32
// entries).
__device__ uint32_t block_scan(uint32_t v, uint32_t *buf, uint32_t &total) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t nw = blockDim.x >> 6;
    const uint32_t incl = wave_incl_scan(v);
    if (lane == 63) buf[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        const uint32_t w = wave_incl_scan(lane < nw ? buf[lane] : 0u);
        if (lane < nw) buf[16 + lane] = w;
    }
    __syncthreads();
    const uint32_t before = wave ? buf[16 + wave - 1] : 0u;
    total = buf[16 + nw - 1];
    __syncthreads();
    return before + incl - v;
}

__device__ __forceinline__ uint32_t block_scan_1024(uint32_t v, uint32_t *buf, uint32_t &total) {
    return block_scan(v, buf, total);
}

// N exclusive block scans behind the same three barriers: v[k] becomes its
// prefix, total[k] the sum (buf[k] needs 32 entries).
template <int N>
__device__ void block_scan_n(uint32_t (&v)[N], uint32_t (*buf)[32], uint32_t (&total)[N]) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t nw = blockDim.x >> 6;
    uint32_t incl[N];
#pragma unroll
    for (int k = 0; k < N; k++) {
        incl[k] = wave_incl_scan(v[k]);
        if (lane == 63) buf[k][wave] = incl[k];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int k = 0; k < N; k++) {
            const uint32_t w = wave_incl_scan(lane < nw ? buf[k][lane] : 0u);
            if (lane < nw) buf[k][16 + lane] = w;
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < N; k++) {
        const uint32_t before = wave ? buf[k][16 + wave - 1] : 0u;
        total[k] = buf[k][16 + nw - 1];
        v[k] = before + incl[k] - v[k];
    }
    __syncthreads();
}

// block_scan of 64-bit values (two packed 32-bit counters scan together
// when neither total overflows); buf needs 32 entries.
__device__ uint64_t block_scan_u64(uint64_t v, uint64_t *buf, uint64_t &total) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t nw = blockDim.x >> 6;
    uint64_t incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint64_t t = __shfl_up(incl, off, 64);
        if (lane >= (uint32_t)off) incl += t;
    }
    if (lane == 63) buf[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        uint64_t w = lane < nw ? buf[lane] : 0ull;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint64_t t = __shfl_up(w, off, 64);
            if (lane >= (uint32_t)off) w += t;
        }
        if (lane < nw) buf[16 + lane] = w;
    }
    __syncthreads();
    const uint64_t before = wave ? buf[16 + wave - 1] : 0ull;
    total = buf[16 + nw - 1];
    __syncthreads();
    return before + incl - v;
}

// One workgroup plans the children of a fused partition + evaluation step
// from the partition's left counts (see launch_level_plan).
// Loads a caller issued early for level_plan_body: the state's counts, the
// totals its last step adds to, and the thread's first pair.
struct PlanPrefetch {
    bool valid;
    uint32_t n, leaf_base, n_eval, hist_nodes;
    uint64_t hist_rows;
    PairDev first;
};

__device__ __forceinline__ void prefetch_state(PlanPrefetch &pre, const GrowState *st) {
    pre.n = st->n_split;
    pre.leaf_base = st->n_leaves;
    pre.n_eval = st->n_eval;
    pre.hist_nodes = st->hist_nodes;
    pre.hist_rows = st->hist_rows;
}

// Sum of v over the block with one barrier: wave sums by shuffles, then
// every thread adds the wave sums. buf holds 16 entries; a caller summing
// again before another barrier passes a different buf.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T *buf) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63u) == 0) buf[threadIdx.x >> 6] = v;
    __syncthreads();
    T t = 0;
    for (uint32_t w = 0; w < (blockDim.x >> 6); w++) t += buf[w];
    return t;
}

__device__ void level_plan_body(const PairDev *pairs, uint32_t n, const uint32_t *totals,
                                ChunkRule rule, HistNodeDev *hn, SplitNodeDev *sn,
                                uint32_t *spans, uint32_t *left_slot, uint32_t *chunk_rows_out,
                                const GrowDevOut &D, const PlanPrefetch &pre) {
    __shared__ uint32_t buf3[3][32];
    __shared__ uint64_t sum64[2][16];
    __shared__ uint32_t sum32[2][16];
    __shared__ uint32_t cr_sh;
    // A device-grown tree: the pair count and the leaf table base come from
    // its state (read by every thread before thread 0 updates it).
    uint32_t leaf_base = 0;
    PlanPrefetch late{};
    if (pre.valid) {
        n = pre.n;
        leaf_base = pre.leaf_base;
    } else if (D.st) {
        prefetch_state(late, D.st);
        n = late.n;
        leaf_base = late.leaf_base;
    }
    const PlanPrefetch &S = pre.valid ? pre : late;
    auto pair_at = [&](uint32_t i) -> PairDev {
        return (pre.valid && i == threadIdx.x) ? pre.first : pairs[i];
    };
    // Spans of every pair and the rows the evaluated pairs accumulate. The
    // thread's first pair (all of them when n <= 1024) stays in registers:
    // left count, and the accumulated (smaller) child's rows when evaluated.
    unsigned long long acc = 0;
    uint32_t my_nl = 0, my_small = 0, nz = 0;
    for (uint32_t i = threadIdx.x; i < n; i += 1024) {
        const PairDev P = pair_at(i);
        const uint32_t nl = P.req == NO_SLOT ? 0u : totals[P.req];
        const uint32_t nr = P.row_len - nl;
        spans[4 * i + 0] = P.row_off;
        spans[4 * i + 1] = nl;
        spans[4 * i + 2] = P.row_off + nl;
        spans[4 * i + 3] = nr;
        const bool ev = P.eval_index != NO_SLOT;
        if (ev) acc += min(nl, nr);
        if (ev && min(nl, nr)) nz++;
        if (i == threadIdx.x) {
            my_nl = nl;
            my_small = ev ? min(nl, nr) : 0u;
        }
    }
    // Accumulated rows of pair i (0 when it is not evaluated).
    auto small_of = [&](uint32_t i) -> uint32_t {
        if (i == threadIdx.x) return my_small;
        const PairDev P = pairs[i];
        if (P.eval_index == NO_SLOT) return 0u;
        const uint32_t nl = P.req == NO_SLOT ? 0u : totals[P.req];
        return min(nl, P.row_len - nl);
    };
    const uint64_t acc_all = block_sum<uint64_t>(acc, sum64[0]);
    const uint32_t n_nz = block_sum<uint32_t>(nz, sum32[0]);  // evaluated pairs whose
                                                                // accumulated child has rows
    unsigned long long acc_nodes = 0;
    // Rows per chunk: the smallest multiple of 1024 whose chunks fit one wave
    // (binary search; each step one block sum of ceil(len / rows)), as the
    // host plans it.
    if (rule.fixed) {
        if (threadIdx.x == 0) cr_sh = rule.fixed;
    } else {
        const uint64_t W = rule.want_chunks;
        uint64_t lo = (acc_all + W * 1024 - 1) / (W * 1024);
        lo = lo < 1 ? 1 : lo;
        if (W > n_nz) {
            const uint64_t room = W - n_nz;
            uint64_t hi = (acc_all + room * 1024 - 1) / (room * 1024);
            hi = hi < lo ? lo : hi;
            uint32_t it = 1;  // sum32[0] was used above
            while (lo < hi) {  // uniform: every thread holds the same bounds
                const uint64_t mid = (lo + hi) / 2, rows = mid * 1024;
                uint32_t k = 0;
                if (rows >> 32) {  // every node with rows takes one chunk
                    for (uint32_t i = threadIdx.x; i < n; i += 1024) k += small_of(i) ? 1u : 0u;
                } else {  // 32-bit divisions: a 64-bit one costs several times more
                    const uint32_t r32 = (uint32_t)rows;
                    for (uint32_t i = threadIdx.x; i < n; i += 1024) {
                        const uint32_t sm = small_of(i);
                        k += sm / r32 + (sm % r32 ? 1u : 0u);
                    }
                }
                const uint32_t total_k = block_sum<uint32_t>(k, sum32[it++ & 1u]);
                if (total_k <= W) hi = mid;
                else lo = mid + 1;
            }
        }
        uint64_t r = lo * 1024;
        r = r < rule.min_rows ? rule.min_rows : (r > rule.max_rows ? rule.max_rows : r);
        if (threadIdx.x == 0) cr_sh = (uint32_t)r;
    }
    __syncthreads();
    if (threadIdx.x == 0) *chunk_rows_out = cr_sh;
    const uint32_t cr = cr_sh;
    uint32_t carry = 0, gcarry = 0;
    for (uint32_t base = 0; base < n; base += 1024) {
        const uint32_t i = base + threadIdx.x;
        PairDev P{};
        uint32_t nl = 0, nr = 0, nc = 0;
        bool ev = false;
        if (i < n) {
            P = pair_at(i);
            ev = P.eval_index != NO_SLOT;
            nl = base == 0 ? my_nl : (P.req == NO_SLOT ? 0u : totals[P.req]);
            nr = P.row_len - nl;
            if (ev) nc = (min(nl, nr) + cr - 1) / cr;
        }
        // Chunks, reduction groups and (children of pairs that are not
        // evaluated are leaves, those with rows) leaves in one scan.
        uint32_t v[3] = {nc, ev && nc >= rule.group_min_chunks ? reduce_groups(nc) : 0u,
                         (D.st && i < n && !ev) ? (nl > 0) + (nr > 0) : 0u};
        uint32_t t[3];
        block_scan_n<3>(v, buf3, t);
        const uint32_t total = t[0], groups_total = t[1], leaves_total = t[2];
        const uint32_t before = carry + v[0];
        const uint32_t group_before = gcarry + v[1];
        const uint32_t leaf_before = leaf_base + v[2];
        if (i < n) {
            // The smaller child (the left one on ties) is accumulated.
            const bool left_small = nl <= nr;
            if (ev) {
                const uint32_t e = P.eval_index;
                HistNodeDev h{};
                h.row_off = left_small ? P.row_off : P.row_off + nl;
                h.row_len = left_small ? nl : nr;
                h.chunk_begin = before;
                h.slot = P.new_slot;
                h.n_chunks = nc;
                h.group_begin = group_before;
                hn[e] = h;
                SplitNodeDev l{}, r{};
                l.sum_g = P.left_sum[0];
                l.sum_h = P.left_sum[1];
                l.lower = P.lower[0];
                l.upper = P.upper[0];
                l.slot = left_small ? P.new_slot : P.parent_slot;
                r.sum_g = P.right_sum[0];
                r.sum_h = P.right_sum[1];
                r.lower = P.lower[1];
                r.upper = P.upper[1];
                r.slot = left_small ? P.parent_slot : P.new_slot;
                sn[2 * e] = l;
                sn[2 * e + 1] = r;
                left_slot[i] = l.slot;
                if (D.st) {
                    LNodeDev a{}, b{};
                    a.tree_id = P.left_id;
                    a.row_off = P.row_off;
                    a.row_len = nl;
                    a.slot = l.slot;
                    a.sum_g = l.sum_g;
                    a.sum_h = l.sum_h;
                    a.lower = l.lower;
                    a.upper = l.upper;
                    b.tree_id = P.right_id;
                    b.row_off = P.row_off + nl;
                    b.row_len = nr;
                    b.slot = r.slot;
                    b.sum_g = r.sum_g;
                    b.sum_h = r.sum_h;
                    b.lower = r.lower;
                    b.upper = r.upper;
                    D.next[2 * e] = a;
                    D.next[2 * e + 1] = b;
                    acc_nodes += min(nl, nr) > 0;
                }
            } else {
                left_slot[i] = NO_SLOT;
                if (D.st) {
                    uint32_t k = leaf_before;
                    const uint32_t ids[2] = {P.left_id, P.right_id};
                    const uint32_t offs[2] = {P.row_off, P.row_off + nl};
                    const uint32_t lens[2] = {nl, nr};
                    for (int c = 0; c < 2; c++) {
                        if (lens[c] == 0) continue;
                        LeafDev lf{};
                        lf.row_off = offs[c];
                        lf.row_len = lens[c];
                        lf.value = D.tree[ids[c]].leaf_value;
                        lf.id = k;
                        lf.arena = D.child_arena;
                        D.leaves[k] = lf;
                        D.leaf_vals[k] = lf.value;
                        D.tree[ids[c]].pad[1] = k;  // the leaf's position
                        k++;
                    }
                }
            }
        }
        carry += total;
        gcarry += groups_total;
        leaf_base += leaves_total;
    }
    if (D.st) {
        // sum64[1]: sum64[0]'s last readers may still be before the scans'
        // barriers above.
        const uint64_t nodes_all = block_sum<uint64_t>(acc_nodes, sum64[1]);
        if (threadIdx.x == 0) {
            GrowState *st = D.st;
            st->n_level = 2 * S.n_eval;
            st->n_leaves = leaf_base;
            st->hist_rows = S.hist_rows + acc_all;
            st->hist_nodes = S.hist_nodes + (uint32_t)nodes_all;
        }
    }
}

__global__ __launch_bounds__(1024) void level_plan_kernel(const PairDev *pairs, uint32_t n,
                                                          const uint32_t *totals, ChunkRule rule,
                                                          HistNodeDev *hn, SplitNodeDev *sn,
                                                          uint32_t *spans, uint32_t *left_slot,
                                                          uint32_t *chunk_rows_out, GrowDevOut D) {
    level_plan_body(pairs, n, totals, rule, hn, sn, spans, left_slot, chunk_rows_out, D,
                    PlanPrefetch{});
}

hipError_t launch_level_plan(const PairDev *pairs, uint32_t n_pairs, const uint32_t *totals,
                             ChunkRule rule, HistNodeDev *hist_nodes, SplitNodeDev *split_nodes,
                             uint32_t *spans, uint32_t *left_slot, uint32_t *chunk_rows,
                             const GrowDevOut &D, hipStream_t s) {
    if (n_pairs == 0 && !D.st) return hipSuccess;
    hipLaunchKernelGGL(level_plan_kernel, dim3(1), dim3(1024), 0, s, pairs, n_pairs, totals, rule,
                       hist_nodes, split_nodes, spans, left_slot, chunk_rows, D);
    return hipGetLastError();
}

// ======================================================================
// split scan
// ======================================================================

constexpr float MIN_GAIN_EPS = 1e-6f;

__device__ __forceinline__ double threshold_l1(double g, float alpha) {
    const double a = (double)alpha;
    if (g > a) return g - a;
    if (g < -a) return g + a;
    return 0.0;
}

// The inverse quantizer scales of the current gradients, from device memory.
__device__ __forceinline__ void load_scales(SplitParamsDev &P) {
    P.inv_g = P.scales->inv[0];
    P.inv_h = P.scales->inv[1];
}

// XGBoost CalcWeight, as split.rs:182-192.
__device__ __forceinline__ float xgb_weight(double g, double h, const SplitParamsDev &P) {
    if (h <= 0.0) return 0.0f;
    double dw = -threshold_l1(g, P.alpha) / (h + (double)P.lambda_);
    if (P.mds != 0.0f && fabs(dw) > (double)P.mds) dw = copysign((double)P.mds, dw);
    return (float)dw;
}

__device__ __forceinline__ float apply_bounds(float w, float lo, float hi) {
    if (w < lo) return lo;
    if (w > hi) return hi;
    return w;
}

// CalcGainGivenWeight, as split.rs:210-218.
__device__ __forceinline__ float gain_given_weight(double g, double h, float w,
                                                   const SplitParamsDev &P) {
    if (h <= 0.0) return 0.0f;
    const float w2 = w * w;
    const double square = (double)w2;
    const double l1 = 2.0 * (double)P.alpha * (double)fabsf(w);
    const double a = 2.0 * g * (double)w;
    const double b = (h + (double)P.lambda_) * square;
    return (float)(-((a + b) + l1));
}

// bounded_split_gain (split.rs:226-252). Returns false when invalid.
__device__ __forceinline__ bool candidate_gain(int64_t lg_i, int64_t lh_i, int64_t rg_i,
                                               int64_t rh_i, float parent, int mono, float lo,
                                               float hi, const SplitParamsDev &P, float &out) {
    const double lg = (double)lg_i * P.inv_g, lh = (double)lh_i * P.inv_h;
    const double rg = (double)rg_i * P.inv_g, rh = (double)rh_i * P.inv_h;
    const double mcw = (double)P.mcw;
    if (!(lh > 0.0 && rh > 0.0 && lh >= mcw && rh >= mcw)) return false;
    const float wl = apply_bounds(xgb_weight(lg, lh, P), lo, hi);
    const float wr = apply_bounds(xgb_weight(rg, rh, P), lo, hi);
    if ((mono > 0 && wl > wr) || (mono < 0 && wl < wr)) return false;
    const float gain = gain_given_weight(lg, lh, wl, P) + gain_given_weight(rg, rh, wr, P);
    const float loss = gain - parent;
    out = (float)((double)loss - (double)P.gamma);
    return true;
}

struct Best {
    float gain;
    uint32_t ord;
    uint32_t found;
    int64_t lg, lh;
};

__device__ __forceinline__ bool better(const Best &a, const Best &b) {
    if (!a.found) return false;
    if (!b.found) return true;
    if (a.gain > b.gain) return true;
    return a.gain == b.gain && a.ord < b.ord;
}

__device__ __forceinline__ void offer(Best &best, float gain, uint32_t ord, int64_t lg,
                                      int64_t lh) {
    // update_best: strict greater than the eps floor and the current best.
    if (!(gain > MIN_GAIN_EPS)) return;
    if (!best.found || gain > best.gain || (gain == best.gain && ord < best.ord)) {
        best.found = 1;
        best.gain = gain;
        best.ord = ord;
        best.lg = lg;
        best.lh = lh;
    }
}

// The best of the wave's candidates by the total order of `better` (gain,
// then the lower ordinal): every lane ends with the same one.
__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        Best o;
        o.gain = __shfl_xor(b.gain, off, 64);
        o.ord = __shfl_xor(b.ord, off, 64);
        o.found = __shfl_xor(b.found, off, 64);
        o.lg = __shfl_xor(b.lg, off, 64);
        o.lh = __shfl_xor(b.lh, off, 64);
        if (better(o, b)) b = o;
    }
    return b;
}

// The block's best by the same order, in every thread: the waves' bests by
// shuffles, then through LDS (sh: one entry a wave).
__device__ Best block_best(Best mine, Best *sh) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const Best w = wave_best(mine);
    if (lane == 0) sh[wave] = w;
    __syncthreads();
    Best r = sh[0];
    for (uint32_t k = 1; k < (blockDim.x >> 6); k++)
        if (better(sh[k], r)) r = sh[k];
    __syncthreads();
    return r;
}

// Inclusive block scan of (g, h) pairs; returns the exclusive prefix of this
// thread and the block total.
__device__ void block_scan_pairs(int64_t g, int64_t h, int64_t *sg, int64_t *shh, int64_t &eg,
                                 int64_t &eh, int64_t &tg, int64_t &th) {
    const uint32_t tid = threadIdx.x;
    sg[tid] = g;
    shh[tid] = h;
    __syncthreads();
    for (uint32_t off = 1; off < SPLIT_TPB; off <<= 1) {
        int64_t ag = 0, ah = 0;
        if (tid >= off) {
            ag = sg[tid - off];
            ah = shh[tid - off];
        }
        __syncthreads();
        sg[tid] = (int64_t)((uint64_t)sg[tid] + (uint64_t)ag);
        shh[tid] = (int64_t)((uint64_t)shh[tid] + (uint64_t)ah);
        __syncthreads();
    }
    eg = (int64_t)((uint64_t)sg[tid] - (uint64_t)g);
    eh = (int64_t)((uint64_t)shh[tid] - (uint64_t)h);
    tg = sg[SPLIT_TPB - 1];
    th = shh[SPLIT_TPB - 1];
    __syncthreads();
}

__device__ __forceinline__ int64_t wadd(int64_t a, int64_t b) {
    return (int64_t)((uint64_t)a + (uint64_t)b);
}
__device__ __forceinline__ int64_t wsub(int64_t a, int64_t b) {
    return (int64_t)((uint64_t)a - (uint64_t)b);
}

// Categorical enumeration of one (node, feature): enumerate_categorical
// (split.rs:484-617). One-hot below max_cat_to_onehot, otherwise a stable
// sort of the categories by weight and prefix scans of at most
// max_cat_threshold - 1 categories per direction.
// Ascending bitonic sort of the 256 * E distinct keys at keys[] (LDS) by
// the workgroup, key q * 256 + t held by thread t in registers: partners
// in the same wave are exchanged by shuffles, those in the same thread
// directly, and only the partners in another wave go through LDS (two
// barriers a step).
template <int E>
__device__ void bitonic_sort_keys(uint64_t *keys) {
    const uint32_t tid = threadIdx.x;
    constexpr uint32_t N2 = E * SPLIT_TPB;
    uint64_t v[E];
#pragma unroll
    for (int q = 0; q < E; q++) v[q] = keys[q * SPLIT_TPB + tid];
    for (uint32_t k = 2; k <= N2; k <<= 1) {
        for (uint32_t jj = k >> 1; jj > 0; jj >>= 1) {
            if (jj >= SPLIT_TPB) {
                const uint32_t d = jj / SPLIT_TPB;
#pragma unroll
                for (int q = 0; q < E; q++) {
                    const uint32_t p = (uint32_t)q ^ d;
                    if (p > (uint32_t)q && p < (uint32_t)E) {
                        const bool up = ((q * SPLIT_TPB + tid) & k) == 0;
                        const uint64_t a = v[q], b = v[p];
                        if ((a > b) == up) {
                            v[q] = b;
                            v[p] = a;
                        }
                    }
                }
            } else if (jj >= 64) {
#pragma unroll
                for (int q = 0; q < E; q++) keys[q * SPLIT_TPB + tid] = v[q];
                __syncthreads();
#pragma unroll
                for (int q = 0; q < E; q++) {
                    const uint32_t i = q * SPLIT_TPB + tid;
                    const uint64_t o = keys[i ^ jj];
                    const bool keep_min = ((i & jj) == 0) == ((i & k) == 0);
                    v[q] = keep_min ? (o < v[q] ? o : v[q]) : (o > v[q] ? o : v[q]);
                }
                __syncthreads();
            } else {
#pragma unroll
                for (int q = 0; q < E; q++) {
                    const uint32_t i = q * SPLIT_TPB + tid;
                    const uint64_t o = __shfl_xor(v[q], (int)jj, 64);
                    const bool keep_min = ((i & jj) == 0) == ((i & k) == 0);
                    v[q] = keep_min ? (o < v[q] ? o : v[q]) : (o > v[q] ? o : v[q]);
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < E; q++) keys[q * SPLIT_TPB + tid] = v[q];
    __syncthreads();
}

__device__ void split_categorical(const int64_t *h, uint32_t n, const SplitNodeDev &N,
                                  float parent, int mono, const SplitParamsDev &P, Best *shb,
                                  int64_t *sg, int64_t *shh, uint64_t *keys, uint32_t *order,
                                  unsigned long long *set_lds, uint64_t *set_out,
                                  uint32_t set_words, FeatCandDev *outc) {
    const uint32_t tid = threadIdx.x;
    int64_t tg = 0, th = 0;
    for (uint32_t i = tid; i < n; i += SPLIT_TPB) {
        tg = wadd(tg, h[2 * i]);
        th = wadd(th, h[2 * i + 1]);
    }
    int64_t eg, eh, totg, toth;
    block_scan_pairs(tg, th, sg, shh, eg, eh, totg, toth);
    const int64_t mg = wsub(N.sum_g, totg), mh = wsub(N.sum_h, toth);  // missing rows

    for (uint32_t w = tid; w < set_words; w += SPLIT_TPB) set_out[w] = 0ull;
    Best best{0.0f, 0u, 0u, 0, 0};
    uint32_t at = 0;
    uint32_t ml = 0;
    if ((uint64_t)n < (uint64_t)P.max_cat_to_onehot) {
        for (uint32_t i = tid; i < n; i += SPLIT_TPB) {
            const int64_t bg = h[2 * i], bh = h[2 * i + 1];
            float gain;
            // Missing rows with the other categories.
            if (candidate_gain(wsub(N.sum_g, bg), wsub(N.sum_h, bh), bg, bh, parent, mono,
                               N.lower, N.upper, P, gain))
                offer(best, gain, 2 * i, wsub(N.sum_g, bg), wsub(N.sum_h, bh));
            // Missing rows with the chosen category.
            const int64_t rg = wadd(bg, mg), rh = wadd(bh, mh);
            if (candidate_gain(wsub(N.sum_g, rg), wsub(N.sum_h, rh), rg, rh, parent, mono,
                               N.lower, N.upper, P, gain))
                offer(best, gain, 2 * i + 1, wsub(N.sum_g, rg), wsub(N.sum_h, rh));
        }
        best = block_best(best, shb);
        if (best.found) {
            at = best.ord >> 1;
            ml = (best.ord & 1) ? 0u : 1u;
        }
        __syncthreads();
        if (tid == 0 && best.found) set_out[at >> 6] |= 1ull << (at & 63);
    } else {
        // Stable ascending order by `<` (std::stable_sort / sort_by
        // partial_cmp): a bitonic sort of (weight, category) keys, the
        // weight's bits mapped so that unsigned order is float order (its
        // zeros made one, as `<` sees them; weights are never NaN) and
        // equal weights ordered by category.
        uint32_t n2 = SPLIT_TPB;
        while (n2 < n) n2 <<= 1;
        for (uint32_t i = tid; i < n2; i += SPLIT_TPB) {
            uint64_t key = ~0ull;  // padding sorts last
            if (i < n) {
                const double g = (double)h[2 * i] * P.inv_g, hh = (double)h[2 * i + 1] * P.inv_h;
                float w = xgb_weight(g, hh, P);
                if (w == 0.0f) w = 0.0f;
                const uint32_t u = __float_as_uint(w);
                key = ((uint64_t)((u & 0x80000000u) ? ~u : (u | 0x80000000u)) << 32) | i;
            }
            keys[i] = key;
        }
        __syncthreads();
        if (n2 == SPLIT_TPB) {
            bitonic_sort_keys<1>(keys);
        } else if (n2 == 2 * SPLIT_TPB) {
            bitonic_sort_keys<2>(keys);
        } else if (n2 == 4 * SPLIT_TPB) {
            bitonic_sort_keys<4>(keys);
        } else {
            for (uint32_t k = 2; k <= n2; k <<= 1)
                for (uint32_t jj = k >> 1; jj > 0; jj >>= 1) {
                    for (uint32_t i = tid; i < n2; i += SPLIT_TPB) {
                        const uint32_t ixj = i ^ jj;
                        if (ixj > i) {
                            const uint64_t a = keys[i], b = keys[ixj];
                            if ((a > b) == ((i & k) == 0)) {
                                keys[i] = b;
                                keys[ixj] = a;
                            }
                        }
                    }
                    __syncthreads();
                }
        }
        // The categories in sorted order; order[] shares the keys' memory,
        // so every key is read before any is overwritten.
        constexpr uint32_t KPT = MAX_DEVICE_CATS / SPLIT_TPB;
        uint32_t cat[KPT];
#pragma unroll
        for (uint32_t q = 0; q < KPT; q++) {
            const uint32_t r = tid + q * SPLIT_TPB;
            cat[q] = r < n ? (uint32_t)keys[r] : 0u;
        }
        __syncthreads();
#pragma unroll
        for (uint32_t q = 0; q < KPT; q++) {
            const uint32_t r = tid + q * SPLIT_TPB;
            if (r < n) order[r] = cat[q];
        }
        __syncthreads();
        const uint32_t n_scan = min(P.max_cat_threshold, n);
        // Prefix sums of the categories in sorted order, each thread a run of
        // them; then every prefix is a candidate in parallel. Forward: the
        // first k+1 categories go right (missing left), ties to the shorter
        // prefix. Backward: categories k..n-1 go left (missing right), ties
        // to the larger k. Integer sums wrap, so T - prefix equals the
        // reference's running suffix exactly.
        const uint32_t per = (n + SPLIT_TPB - 1) / SPLIT_TPB;
        const uint32_t k0 = min(tid * per, n), k1 = min(k0 + per, n);
        int64_t sg_loc = 0, sh_loc = 0;
        for (uint32_t k = k0; k < k1; k++) {
            sg_loc = wadd(sg_loc, h[2 * order[k]]);
            sh_loc = wadd(sh_loc, h[2 * order[k] + 1]);
        }
        int64_t exg, exh, allg, allh;
        block_scan_pairs(sg_loc, sh_loc, sg, shh, exg, exh, allg, allh);
        Best fwd{0.0f, 0u, 0u, 0, 0}, bwd{0.0f, 0u, 0u, 0, 0};
        if (n_scan >= 2) {
            int64_t cg = exg, ch = exh;  // sum of the categories before k
            for (uint32_t k = k0; k < k1; k++) {
                float gain;
                if (k >= n - (n_scan - 1)) {
                    const int64_t lg = wsub(allg, cg), lh = wsub(allh, ch);
                    const int64_t rg = wsub(N.sum_g, lg), rh = wsub(N.sum_h, lh);
                    if (candidate_gain(lg, lh, rg, rh, parent, mono, N.lower, N.upper, P, gain))
                        offer(bwd, gain, n - 1 - k, lg, lh);
                }
                cg = wadd(cg, h[2 * order[k]]);
                ch = wadd(ch, h[2 * order[k] + 1]);
                if (k + 1 < n_scan) {
                    const int64_t lg = wsub(N.sum_g, cg), lh = wsub(N.sum_h, ch);
                    if (candidate_gain(lg, lh, cg, ch, parent, mono, N.lower, N.upper, P, gain))
                        offer(fwd, gain, k + 1, lg, lh);
                }
            }
        }
        fwd = block_best(fwd, shb);
        bwd = block_best(bwd, shb);
        best = fwd;
        ml = 1;
        at = fwd.ord;
        if (bwd.found && (!fwd.found || bwd.gain > fwd.gain)) {
            best = bwd;
            ml = 0;
            at = n - 1 - bwd.ord;
        }
        // The right-going set: the first `at` categories in sorted order.
        for (uint32_t w = tid; w < set_words; w += SPLIT_TPB) set_lds[w] = 0ull;
        __syncthreads();
        if (best.found)
            for (uint32_t kk = tid; kk < at; kk += SPLIT_TPB)
                atomicOr(&set_lds[order[kk] >> 6], 1ull << (order[kk] & 63));
        __syncthreads();
        for (uint32_t w = tid; w < set_words; w += SPLIT_TPB) set_out[w] = set_lds[w];
    }
    if (tid == 0) {
        outc->found = best.found;
        outc->gain = best.gain;
        outc->bin = 0;
        outc->missing_left = ml;
        outc->left_g = best.lg;
        outc->left_h = best.lh;
    }
}

__device__ __forceinline__ int64_t wave_scan_incl_i64(int64_t v, uint32_t lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int64_t t = __shfl_up(v, off, 64);
        if (lane >= (uint32_t)off) v = wadd(v, t);
    }
    return v;
}


// One wave per (numeric feature, node), four features per workgroup: the
// numeric scan of split_feat_kernel on 64 lanes with shuffles only (no
// barriers). Each lane takes a run of bins; integer prefix sums are exact in
// any order, and the argmax keeps the reference's tie rule.
// Bins of a numeric feature held in registers: lane l of a wave (thread t
// of a workgroup) holds bins [l * per, l * per + per), per = ceil(bins / 64)
// (ceil(bins / 256)) at most NUM_PER_LANE: one wave for features of at most
// 256 bins, four for those of at most 1024.
constexpr uint32_t NUM_PER_LANE = 4;

// The node's gain before the split (the parent term of every candidate).
__device__ __forceinline__ float parent_gain(const SplitNodeDev &N, const SplitParamsDev &P) {
    const double ng = (double)N.sum_g * P.inv_g, nh = (double)N.sum_h * P.inv_h;
    return gain_given_weight(ng, nh, apply_bounds(xgb_weight(ng, nh, P), N.lower, N.upper), P);
}

// The lane's candidates of a numeric scan over its bins (g[k], h[k] of bin
// b0 + k, summing to tg, th): the forward ones (missing rows right) from
// eg, eh, the sums of the feature's bins before b0, and the reverse ones
// (missing rows left; skipped when the feature's bins, totg / toth, hold the
// whole node). Returns the lane's first best by the reference's rules.
template <uint32_t PER>
__device__ __forceinline__ Best scan_candidates(const int64_t (&g)[PER], const int64_t (&h)[PER],
                                                uint32_t b0, uint32_t b1, uint32_t n,
                                                const SplitNodeDev &N, int mono,
                                                const SplitParamsDev &P, float parent, int64_t tg,
                                                int64_t th, int64_t eg, int64_t eh, int64_t totg,
                                                int64_t toth) {
    Best best{0.0f, 0u, 0u, 0, 0};
    // Forward: missing rows go right.
    int64_t lg = eg, lh = eh;
#pragma unroll
    for (uint32_t k = 0; k < PER; k++) {
        if (b0 + k >= b1) break;
        lg = wadd(lg, g[k]);
        lh = wadd(lh, h[k]);
        float gain;
        if (candidate_gain(lg, lh, wsub(N.sum_g, lg), wsub(N.sum_h, lh), parent, mono, N.lower,
                           N.upper, P, gain))
            offer(best, gain, b0 + k, lg, lh);
    }
    // Reverse: missing rows go left; skipped when the bins hold the whole node.
    if (!(totg == N.sum_g && toth == N.sum_h)) {
        int64_t rg = wsub(wsub(totg, eg), tg), rh = wsub(wsub(toth, eh), th);
#pragma unroll
        for (int k = PER - 1; k >= 0; k--) {
            if (b0 + k >= b1) continue;
            rg = wadd(rg, g[k]);
            rh = wadd(rh, h[k]);
            const int64_t l2g = wsub(N.sum_g, rg), l2h = wsub(N.sum_h, rh);
            float gain;
            if (candidate_gain(l2g, l2h, rg, rh, parent, mono, N.lower, N.upper, P, gain))
                offer(best, gain, n + (n - 1 - (b0 + k)), l2g, l2h);
        }
    }
    return best;
}

// A numeric scan's best into its candidate slot (ordinals below n: bin + 1
// with missing rows right; above: the reverse scan's, missing rows left).
__device__ __forceinline__ void write_numeric_cand(const Best &best, uint32_t n,
                                                   FeatCandDev *outc) {
    outc->found = best.found;
    outc->gain = best.gain;
    if (best.ord < n) {
        outc->bin = best.ord + 1;
        outc->missing_left = 0;
    } else {
        outc->bin = n - 1 - (best.ord - n);
        outc->missing_left = 1;
    }
    outc->left_g = best.lg;
    outc->left_h = best.lh;
}

// The split scan of one (node, feature) over bins in the wave's registers:
// prefix sums by shuffles, the lanes' candidates, the wave's first best,
// written to outc by lane 0.
template <uint32_t PER>
__device__ __forceinline__ void scan_numeric(const int64_t (&g)[PER], const int64_t (&h)[PER],
                                             uint32_t b0, uint32_t b1, uint32_t n, uint32_t lane,
                                             const SplitNodeDev &N, const SplitFeatDev &F,
                                             const SplitParamsDev &P, FeatCandDev *outc) {
    const float parent = parent_gain(N, P);
    int64_t tg = 0, th = 0;
#pragma unroll
    for (uint32_t k = 0; k < PER; k++)
        if (b0 + k < b1) {
            tg = wadd(tg, g[k]);
            th = wadd(th, h[k]);
        }
    const int64_t ig = wave_scan_incl_i64(tg, lane), ih = wave_scan_incl_i64(th, lane);
    const int64_t totg = __shfl(ig, 63, 64), toth = __shfl(ih, 63, 64);
    Best best = scan_candidates<PER>(g, h, b0, b1, n, N, F.monotone, P, parent, tg, th,
                                     wsub(ig, tg), wsub(ih, th), totg, toth);
    best = wave_best(best);
    if (lane == 0) write_numeric_cand(best, n, outc);
}

// One wave's (node, numeric feature of at most 64 * PER bins): the
// feature's bins into registers, then scan_numeric. li indexes order.
// triples set (sibling subtraction fused, nodes 2e and 2e + 1 the children
// of evaluated pair e): the larger child took its parent's slot, which
// still holds the parent's histogram, so its bins are those minus the
// smaller child's (slot triples[3e + 2]), stored back when write_big (the
// next level's parents), whether or not the feature is enabled here.
template <uint32_t PER>
__device__ __forceinline__ void split_num_wave(int64_t *hist, uint64_t hist_width,
                                               const SplitNodeDev *nodes,
                                               const SplitFeatDev *feats, const uint32_t *order,
                                               uint32_t li, uint32_t ni, const uint8_t *enabled,
                                               SplitParamsDev P, FeatCandDev *cands,
                                               const uint32_t *triples, uint32_t write_big) {
    const uint32_t lane = threadIdx.x & 63u;
    load_scales(P);
    const uint32_t j = order[li];
    const SplitFeatDev F = feats[j];
    const SplitNodeDev N = nodes[ni];
    const uint32_t small_slot = triples ? triples[3 * (ni >> 1) + 2] : NO_SLOT;
    const bool big = triples && N.slot != small_slot;
    FeatCandDev *outc = cands + (size_t)ni * P.n_feats + j;
    const bool off = enabled && !enabled[(size_t)ni * P.n_feats + j];
    if (off && !big) {
        if (lane == 0) outc->found = 0;
        return;
    }
    int64_t *hp = hist + ((uint64_t)N.slot * hist_width + F.hist_off) * 2u;
    const uint32_t n = F.n_bins;
    const uint32_t per = (n + 63) / 64;  // at most PER
    const uint32_t b0 = min(lane * per, n), b1 = min(b0 + per, n);
    int64_t g[PER], h[PER];
#pragma unroll
    for (uint32_t k = 0; k < PER; k++) {
        g[k] = b0 + k < b1 ? hp[2 * (b0 + k)] : 0;
        h[k] = b0 + k < b1 ? hp[2 * (b0 + k) + 1] : 0;
    }
    if (big) {
        const int64_t *sp = hist + ((uint64_t)small_slot * hist_width + F.hist_off) * 2u;
#pragma unroll
        for (uint32_t k = 0; k < PER; k++)
            if (b0 + k < b1) {
                g[k] = wsub(g[k], sp[2 * (b0 + k)]);
                h[k] = wsub(h[k], sp[2 * (b0 + k) + 1]);
                if (write_big) {
                    hp[2 * (b0 + k)] = g[k];
                    hp[2 * (b0 + k) + 1] = h[k];
                }
            }
        if (off) {
            if (lane == 0) outc->found = 0;
            return;
        }
    }
    scan_numeric<PER>(g, h, b0, b1, n, lane, N, F, P, outc);
}

// One workgroup's (node, numeric feature of 257 to 1024 bins): each of its
// four waves holds a quarter of the bins in registers (at most four a
// lane), the waves' sums are exchanged through LDS for the prefix and the
// total, every lane scans its candidates, and the waves' bests are combined
// by the same total order. Four waves a feature keep the chain of f64
// candidate arithmetic a lane runs four times shorter than one wave would.
// wt holds 8 and wb 4 entries of LDS. li indexes order.
__device__ __forceinline__ void split_wide_block(int64_t *hist, uint64_t hist_width,
                                                 const SplitNodeDev *nodes,
                                                 const SplitFeatDev *feats, const uint32_t *order,
                                                 uint32_t li, uint32_t ni, const uint8_t *enabled,
                                                 SplitParamsDev P, FeatCandDev *cands,
                                                 int64_t *wt, Best *wb, const uint32_t *triples,
                                                 uint32_t write_big) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    load_scales(P);
    const uint32_t j = order[li];
    const SplitFeatDev F = feats[j];
    const SplitNodeDev N = nodes[ni];
    FeatCandDev *outc = cands + (size_t)ni * P.n_feats + j;
    // Sibling subtraction in registers (triples set), as split_num_wave.
    const uint32_t small_slot = triples ? triples[3 * (ni >> 1) + 2] : NO_SLOT;
    const bool big = triples && N.slot != small_slot;
    const bool off = enabled && !enabled[(size_t)ni * P.n_feats + j];
    if (off && !big) {
        if (tid == 0) outc->found = 0;
        return;
    }
    int64_t *hp = hist + ((uint64_t)N.slot * hist_width + F.hist_off) * 2u;
    const uint32_t n = F.n_bins;
    const uint32_t per = (n + SPLIT_TPB - 1) / SPLIT_TPB;  // at most NUM_PER_LANE
    const uint32_t b0 = min(tid * per, n), b1 = min(b0 + per, n);
    int64_t g[NUM_PER_LANE], h[NUM_PER_LANE];
#pragma unroll
    for (uint32_t k = 0; k < NUM_PER_LANE; k++) {
        g[k] = b0 + k < b1 ? hp[2 * (b0 + k)] : 0;
        h[k] = b0 + k < b1 ? hp[2 * (b0 + k) + 1] : 0;
    }
    if (big) {
        const int64_t *sp = hist + ((uint64_t)small_slot * hist_width + F.hist_off) * 2u;
#pragma unroll
        for (uint32_t k = 0; k < NUM_PER_LANE; k++)
            if (b0 + k < b1) {
                g[k] = wsub(g[k], sp[2 * (b0 + k)]);
                h[k] = wsub(h[k], sp[2 * (b0 + k) + 1]);
                if (write_big) {
                    hp[2 * (b0 + k)] = g[k];
                    hp[2 * (b0 + k) + 1] = h[k];
                }
            }
        if (off) {
            if (tid == 0) outc->found = 0;
            return;
        }
    }
    int64_t tg = 0, th = 0;
#pragma unroll
    for (uint32_t k = 0; k < NUM_PER_LANE; k++) {
        tg = wadd(tg, g[k]);
        th = wadd(th, h[k]);
    }
    const int64_t ig = wave_scan_incl_i64(tg, lane), ih = wave_scan_incl_i64(th, lane);
    if (lane == 63) {
        wt[2 * wave] = ig;
        wt[2 * wave + 1] = ih;
    }
    __syncthreads();
    int64_t og = 0, oh = 0, totg = 0, toth = 0;
    for (uint32_t w = 0; w < SPLIT_TPB / 64; w++) {
        if (w < wave) {
            og = wadd(og, wt[2 * w]);
            oh = wadd(oh, wt[2 * w + 1]);
        }
        totg = wadd(totg, wt[2 * w]);
        toth = wadd(toth, wt[2 * w + 1]);
    }
    Best best = scan_candidates<NUM_PER_LANE>(g, h, b0, b1, n, N, F.monotone, P, parent_gain(N, P),
                                              tg, th, wadd(og, wsub(ig, tg)),
                                              wadd(oh, wsub(ih, th)), totg, toth);
    best = wave_best(best);
    if (lane == 0) wb[wave] = best;
    __syncthreads();
    if (tid == 0) {
        Best b = wb[0];
        for (uint32_t w = 1; w < SPLIT_TPB / 64; w++)
            if (better(wb[w], b)) b = wb[w];
        write_numeric_cand(b, n, outc);
    }
}

// One wave per (node, numeric feature of at most 256 bins), four features a
// workgroup.
__global__ __launch_bounds__(256) void split_num_kernel(
    int64_t *hist, uint64_t hist_width, const SplitNodeDev *nodes, const SplitFeatDev *feats,
    const uint32_t *order, uint32_t n_num, const uint8_t *enabled, SplitParamsDev P,
    FeatCandDev *cands, const uint32_t *dev_n, const uint32_t *triples, uint32_t write_big) {
    const uint32_t li = blockIdx.x * 4 + (threadIdx.x >> 6), ni = blockIdx.y;
    if (dev_n && ni >= *dev_n) return;
    if (li >= n_num) return;  // a whole wave
    split_num_wave<NUM_PER_LANE>(hist, hist_width, nodes, feats, order, li, ni, enabled, P, cands,
                                 triples, write_big);
}

// Reduction, subtraction and split scan of one evaluated pair in one pass,
// one wave per (pair, numeric feature of at most 256 bins): the accumulated
// (smaller) child's bins come from its chunks' partials when it has 2 to
// PAIR_MAX_CHUNKS chunks, else from its slot (one chunk: stored by the
// histogram launch; more: summed there by reduce_chunks_kernel; none: zeros);
// the larger child's are the parent's minus those. Both children's bins are
// stored to their slots (the larger in place of the parent's) when `write`
// (they are parents at the next level), and both are scanned. Pair e holds
// hn[e] (the accumulated child), triples[3e..3e+2] (larger child's slot,
// parent slot, accumulated slot) and nodes 2e, 2e + 1 (left, right).
__global__ __launch_bounds__(256) void split_pair_kernel(
    int64_t *hist, uint64_t hist_width, const int64_t *partials, const HistNodeDev *hn,
    const uint32_t *triples, const SplitNodeDev *nodes, const SplitFeatDev *feats,
    const uint32_t *order, uint32_t n_num, const uint8_t *enabled, SplitParamsDev P,
    FeatCandDev *cands, const uint32_t *dev_n, uint32_t write) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t li = blockIdx.x * 4 + wave, e = blockIdx.y;
    if (dev_n && e >= *dev_n) return;
    if (li >= n_num) return;  // a whole wave
    load_scales(P);
    const uint32_t j = order[li];
    const SplitFeatDev F = feats[j];
    const HistNodeDev H = hn[e];
    const uint32_t big_slot = triples[3 * e], par_slot = triples[3 * e + 1];
    const uint64_t W = hist_width * 2u;
    const uint32_t n = F.n_bins;
    const uint32_t per = (n + 63) / 64;  // at most NUM_PER_LANE
    const uint32_t b0 = min(lane * per, n), b1 = min(b0 + per, n);
    const uint64_t off = 2u * (uint64_t)F.hist_off;
    int64_t sg[NUM_PER_LANE], sh[NUM_PER_LANE];
    const bool from_partials = partials && H.n_chunks > 1 && H.n_chunks <= PAIR_MAX_CHUNKS;
    if (from_partials) {
#pragma unroll
        for (uint32_t k = 0; k < NUM_PER_LANE; k++) sg[k] = sh[k] = 0;
        // Four chunks' loads in flight at a time (a chunk past the node's
        // reads its first chunk again and adds nothing).
        for (uint32_t c = 0; c < H.n_chunks; c += 4) {
            int64_t vg[4][NUM_PER_LANE], vh[4][NUM_PER_LANE];
#pragma unroll
            for (uint32_t q = 0; q < 4; q++) {
                const uint32_t cc = c + q < H.n_chunks ? c + q : 0u;
                const int64_t *pp = partials + (uint64_t)(H.chunk_begin + cc) * W + off;
#pragma unroll
                for (uint32_t k = 0; k < NUM_PER_LANE; k++) {
                    vg[q][k] = b0 + k < b1 ? pp[2 * (b0 + k)] : 0;
                    vh[q][k] = b0 + k < b1 ? pp[2 * (b0 + k) + 1] : 0;
                }
            }
#pragma unroll
            for (uint32_t q = 0; q < 4; q++)
                if (c + q < H.n_chunks) {
#pragma unroll
                    for (uint32_t k = 0; k < NUM_PER_LANE; k++) {
                        sg[k] = wadd(sg[k], vg[q][k]);
                        sh[k] = wadd(sh[k], vh[q][k]);
                    }
                }
        }
    } else {
        const int64_t *sp = hist + (uint64_t)H.slot * W + off;
#pragma unroll
        for (uint32_t k = 0; k < NUM_PER_LANE; k++) {
            const bool in = H.n_chunks && b0 + k < b1;
            sg[k] = in ? sp[2 * (b0 + k)] : 0;
            sh[k] = in ? sp[2 * (b0 + k) + 1] : 0;
        }
    }
    int64_t bg[NUM_PER_LANE], bh[NUM_PER_LANE];
    {
        const int64_t *pp = hist + (uint64_t)par_slot * W + off;
#pragma unroll
        for (uint32_t k = 0; k < NUM_PER_LANE; k++) {
            bg[k] = b0 + k < b1 ? wsub(pp[2 * (b0 + k)], sg[k]) : 0;
            bh[k] = b0 + k < b1 ? wsub(pp[2 * (b0 + k) + 1], sh[k]) : 0;
        }
    }
    if (write) {
        int64_t *bp = hist + (uint64_t)big_slot * W + off;
        int64_t *sp = hist + (uint64_t)H.slot * W + off;
        const bool store_small = from_partials || H.n_chunks == 0;
#pragma unroll
        for (uint32_t k = 0; k < NUM_PER_LANE; k++)
            if (b0 + k < b1) {
                bp[2 * (b0 + k)] = bg[k];
                bp[2 * (b0 + k) + 1] = bh[k];
                if (store_small) {
                    sp[2 * (b0 + k)] = sg[k];
                    sp[2 * (b0 + k) + 1] = sh[k];
                }
            }
    }
    // One copy of the scan for both children: with two, the kernel's code
    // outgrows the instruction cache (400k x 2000 rounds 5-24: 382 -> 390
    // rounds/s).
#pragma unroll 1
    for (uint32_t side = 0; side < 2; side++) {
        const uint32_t ni = 2 * e + side;
        const SplitNodeDev N = nodes[ni];
        FeatCandDev *outc = cands + (size_t)ni * P.n_feats + j;
        if (enabled && !enabled[(size_t)ni * P.n_feats + j]) {
            if (lane == 0) outc->found = 0;
            continue;
        }
        const bool small = N.slot == H.slot;
        int64_t xg[NUM_PER_LANE], xh[NUM_PER_LANE];
#pragma unroll
        for (uint32_t k = 0; k < NUM_PER_LANE; k++) {
            xg[k] = small ? sg[k] : bg[k];
            xh[k] = small ? sh[k] : bh[k];
        }
        scan_numeric<NUM_PER_LANE>(xg, xh, b0, b1, n, lane, N, F, P, outc);
    }
}

hipError_t launch_split_pairs(int64_t *hist, uint64_t hist_width, const int64_t *partials,
                              const HistNodeDev *hn, const uint32_t *triples, uint32_t n_pairs,
                              const SplitNodeDev *nodes, const SplitFeatDev *feats,
                              const uint32_t *order, uint32_t n_num, const uint8_t *enabled,
                              SplitParamsDev P, FeatCandDev *cands, const uint32_t *dev_n,
                              bool write, hipStream_t s) {
    if (n_pairs == 0 || n_num == 0) return hipSuccess;
    hipLaunchKernelGGL(split_pair_kernel, dim3((n_num + 3) / 4, n_pairs), dim3(256), 0, s, hist,
                       hist_width, partials, hn, triples, nodes, feats, order, n_num, enabled, P,
                       cands, dev_n, write ? 1u : 0u);
    return hipGetLastError();
}

// One workgroup per (feature, node): prefix sums of the feature's bins, the
// forward (missing right) and reverse (missing left, only when the node has
// missing mass) candidates, and the first best by the reference's rules.
// Workgroups past the n_block one-workgroup features take the n_wide
// numeric features of at most 1024 bins that follow order[wide_off], one
// workgroup each (split_wide_block), in the same launch: the two kinds then
// overlap instead of running one after the other.
__global__ __launch_bounds__(SPLIT_TPB) void split_feat_kernel(
    int64_t *hist, uint64_t hist_width, const SplitNodeDev *nodes, const SplitFeatDev *feats,
    const uint32_t *order, uint32_t order_off, uint32_t n_block, uint32_t wide_off,
    uint32_t n_wide, const uint8_t *enabled, SplitParamsDev P, FeatCandDev *cands,
    uint64_t *cat_scratch, const uint32_t *dev_n, const uint32_t *triples, uint32_t write_big) {
    __shared__ Best shb[SPLIT_TPB];
    __shared__ int64_t sg[SPLIT_TPB], shh[SPLIT_TPB];
    extern __shared__ unsigned char dyn[];

    const uint32_t ni = blockIdx.y, tid = threadIdx.x;
    if (dev_n && ni >= *dev_n) return;
    if (blockIdx.x >= n_block) {
        const uint32_t li = blockIdx.x - n_block;
        if (li < n_wide)
            split_wide_block(hist, hist_width, nodes, feats, order + wide_off, li, ni, enabled, P,
                             cands, sg, shb, triples, write_big);
        return;
    }
    load_scales(P);
    const uint32_t j = order[order_off + blockIdx.x];
    const SplitFeatDev F = feats[j];
    const SplitNodeDev N = nodes[ni];
    FeatCandDev *outc = cands + (size_t)ni * P.n_feats + j;
    // Sibling subtraction (triples set), as split_num_wave: the larger child's
    // bins, its parent's minus the smaller child's, are stored into its slot
    // first (the scans below read them from there), enabled or not.
    const uint32_t small_slot = triples ? triples[3 * (ni >> 1) + 2] : NO_SLOT;
    const bool big = triples && N.slot != small_slot;
    const bool off = enabled && !enabled[(size_t)ni * P.n_feats + j];
    if (off && !big) {
        if (tid == 0) outc->found = 0;
        return;
    }
    int64_t *hm = hist + ((uint64_t)N.slot * hist_width + F.hist_off) * 2u;
    if (big) {
        const int64_t *sp = hist + ((uint64_t)small_slot * hist_width + F.hist_off) * 2u;
        for (uint32_t i = tid; i < 2 * F.n_bins; i += SPLIT_TPB) hm[i] = wsub(hm[i], sp[i]);
        __threadfence_block();
        __syncthreads();
        if (off) {
            if (tid == 0) outc->found = 0;
            return;
        }
    }
    const int64_t *h = hm;
    const double ng = (double)N.sum_g * P.inv_g, nh = (double)N.sum_h * P.inv_h;
    const float parent = gain_given_weight(ng, nh, apply_bounds(xgb_weight(ng, nh, P), N.lower,
                                                                N.upper), P);
    const uint32_t n = F.n_bins;

    if (F.categorical) {
        // Sort keys (8 bytes a category), then the sorted categories in the
        // same memory.
        uint64_t *keys = reinterpret_cast<uint64_t *>(dyn);
        uint32_t *order = reinterpret_cast<uint32_t *>(dyn);
        uint64_t *set = cat_scratch + (size_t)ni * P.cat_words_per_node + F.cat_base;
        __shared__ unsigned long long set_lds[MAX_DEVICE_CATS / 64];
        split_categorical(h, n, N, parent, F.monotone, P, shb, sg, shh, keys, order, set_lds, set,
                          F.cat_words, outc);
        return;
    }

    const uint32_t per = (n + SPLIT_TPB - 1) / SPLIT_TPB;
    const uint32_t b0 = min(tid * per, n), b1 = min(b0 + per, n);
    int64_t tg = 0, th = 0;
    for (uint32_t bb = b0; bb < b1; bb++) {
        tg = wadd(tg, h[2 * bb]);
        th = wadd(th, h[2 * bb + 1]);
    }
    int64_t eg, eh, totg, toth;
    block_scan_pairs(tg, th, sg, shh, eg, eh, totg, toth);

    Best best{0.0f, 0u, 0u, 0, 0};
    const int mono = F.monotone;
    // Forward: missing rows go right.
    int64_t lg = eg, lh = eh;
    for (uint32_t bb = b0; bb < b1; bb++) {
        lg = wadd(lg, h[2 * bb]);
        lh = wadd(lh, h[2 * bb + 1]);
        float gain;
        if (candidate_gain(lg, lh, wsub(N.sum_g, lg), wsub(N.sum_h, lh), parent, mono, N.lower,
                           N.upper, P, gain))
            offer(best, gain, bb, lg, lh);
    }
    // Reverse: missing rows go left; skipped when the bins hold the whole node.
    if (!(totg == N.sum_g && toth == N.sum_h)) {
        // Sum of the bins after this thread's range.
        int64_t rg = wsub(wsub(totg, eg), tg), rh = wsub(wsub(toth, eh), th);
        for (uint32_t bb = b1; bb-- > b0;) {
            rg = wadd(rg, h[2 * bb]);
            rh = wadd(rh, h[2 * bb + 1]);
            const int64_t l2g = wsub(N.sum_g, rg), l2h = wsub(N.sum_h, rh);
            float gain;
            if (candidate_gain(l2g, l2h, rg, rh, parent, mono, N.lower, N.upper, P, gain))
                offer(best, gain, n + (n - 1 - bb), l2g, l2h);
        }
    }
    best = block_best(best, shb);
    if (tid == 0) {
        outc->found = best.found;
        outc->gain = best.gain;
        if (best.ord < n) {
            outc->bin = best.ord + 1;
            outc->missing_left = 0;
        } else {
            outc->bin = n - 1 - (best.ord - n);
            outc->missing_left = 1;
        }
        outc->left_g = best.lg;
        outc->left_h = best.lh;
    }
}

hipError_t launch_split_feats(int64_t *hist, uint64_t hist_width, const SplitNodeDev *nodes,
                              uint32_t n_nodes, const SplitFeatDev *feats, const uint32_t *order,
                              uint32_t n_num, uint32_t n_wide, uint32_t n_cat,
                              const uint8_t *enabled, SplitParamsDev P, FeatCandDev *cands,
                              uint64_t *cat_scratch, const uint32_t *dev_n,
                              const uint32_t *sub_triples, bool write_big, hipStream_t s) {
    if (n_nodes == 0 || P.n_feats == 0) return hipSuccess;
    if (n_num)
        hipLaunchKernelGGL(split_num_kernel, dim3((n_num + 3) / 4, n_nodes), dim3(256), 0, s, hist,
                           hist_width, nodes, feats, order, n_num, enabled, P, cands, dev_n,
                           sub_triples, write_big ? 1u : 0u);
    if (n_wide || n_cat) {
        const size_t dyn = P.cat_words_per_node
                               ? sizeof(uint64_t) * MAX_DEVICE_CATS
                               : 0;
        hipLaunchKernelGGL(split_feat_kernel, dim3(n_cat + n_wide, n_nodes),
                           dim3(SPLIT_TPB), dyn, s, hist, hist_width, nodes, feats, order,
                           n_num + n_wide, n_cat, n_num, n_wide, enabled, P, cands, cat_scratch,
                           dev_n, sub_triples, write_big ? 1u : 0u);
    }
    return hipGetLastError();
}

// Per node: the best feature by gain, ties to the lowest feature id
// (features are in ascending global order), as reduce_best / update_best.
// The packet of node ni whose best feature (in split-scan order) is ord;
// a categorical winner's category set is copied to cat_out.
__device__ SplitPacketDev split_packet(const FeatCandDev *c, const SplitFeatDev *feats,
                                       const SplitParamsDev &P, uint32_t ni, uint32_t found,
                                       uint32_t ord, const SplitNodeDev *nodes,
                                       const uint64_t *cat_scratch, uint64_t *cat_out,
                                       uint32_t cat_out_words) {
    SplitPacketDev pk;
    pk.found = found;
    pk.feat = 0;
    pk.bin = 0;
    pk.missing_left = 0;
    pk.gain = 0.0f;
    pk.is_cat = 0;
    pk.cat_offset = ni * cat_out_words;
    pk.n_cat_words = 0;
    pk.left[0] = pk.left[1] = pk.right[0] = pk.right[1] = 0;
    if (found) {
        const FeatCandDev w = c[ord];
        const SplitFeatDev F = feats[ord];
        const SplitNodeDev N = nodes[ni];
        pk.feat = F.feat;
        pk.bin = w.bin;
        pk.missing_left = w.missing_left;
        pk.gain = w.gain;
        pk.left[0] = w.left_g;
        pk.left[1] = w.left_h;
        pk.right[0] = wsub(N.sum_g, w.left_g);
        pk.right[1] = wsub(N.sum_h, w.left_h);
        if (F.categorical) {
            pk.is_cat = 1;
            pk.n_cat_words = F.cat_words;
            const uint64_t *src = cat_scratch + (size_t)ni * P.cat_words_per_node + F.cat_base;
            for (uint32_t k = 0; k < F.cat_words && k < cat_out_words; k++)
                cat_out[(size_t)ni * cat_out_words + k] = src[k];
        }
    }
    return pk;
}

// The packet of node ni from its candidates by one thread: the first
// feature of the largest gain, as block_best picks it (found candidates
// have gains above MIN_GAIN_EPS, never NaN).
__device__ SplitPacketDev split_packet_serial(const FeatCandDev *cands, const SplitFeatDev *feats,
                                              const SplitParamsDev &P, uint32_t ni,
                                              const SplitNodeDev *nodes,
                                              const uint64_t *cat_scratch, uint64_t *cat_out,
                                              uint32_t cat_out_words) {
    const FeatCandDev *c = cands + (size_t)ni * P.n_feats;
    uint32_t found = 0, ord = 0;
    float gain = 0.0f;
    uint32_t j = 0;
    // Eight candidates' loads in flight at a time.
    for (; j + 8 <= P.n_feats; j += 8) {
        float gj[8];
        uint32_t fj[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            gj[k] = c[j + k].gain;
            fj[k] = c[j + k].found;
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (fj[k] && (!found || gj[k] > gain)) {
                found = 1;
                gain = gj[k];
                ord = j + k;
            }
    }
    for (; j < P.n_feats; j++) {
        const FeatCandDev cj = c[j];
        if (cj.found && (!found || cj.gain > gain)) {
            found = 1;
            gain = cj.gain;
            ord = j;
        }
    }
    return split_packet(c, feats, P, ni, found, ord, nodes, cat_scratch, cat_out, cat_out_words);
}

__global__ __launch_bounds__(SPLIT_TPB) void split_node_kernel(
    const FeatCandDev *cands, const SplitFeatDev *feats, SplitParamsDev P,
    const SplitNodeDev *nodes, const uint64_t *cat_scratch, SplitPacketDev *out,
    uint64_t *cat_out, uint32_t cat_out_words, const uint32_t *dev_n) {
    __shared__ Best shb[SPLIT_TPB];
    const uint32_t ni = blockIdx.x, tid = threadIdx.x;
    if (dev_n && ni >= *dev_n) return;
    load_scales(P);
    const FeatCandDev *c = cands + (size_t)ni * P.n_feats;
    Best best{0.0f, 0u, 0u, 0, 0};
    for (uint32_t j = tid; j < P.n_feats; j += SPLIT_TPB) {
        const FeatCandDev cj = c[j];
        if (cj.found && (!best.found || cj.gain > best.gain)) {
            best.found = 1;
            best.gain = cj.gain;
            best.ord = j;
        }
    }
    best = block_best(best, shb);
    if (tid == 0)
        out[ni] = split_packet(c, feats, P, ni, best.found, best.ord, nodes, cat_scratch, cat_out,
                               cat_out_words);
}

hipError_t launch_split_nodes(const FeatCandDev *cands, const SplitFeatDev *feats,
                              uint32_t n_nodes, SplitParamsDev P, const SplitNodeDev *nodes,
                              const uint64_t *cat_scratch, SplitPacketDev *out,
                              uint64_t *cat_out, uint32_t cat_out_words, const uint32_t *dev_n,
                              hipStream_t s) {
    if (n_nodes == 0) return hipSuccess;
    hipLaunchKernelGGL(split_node_kernel, dim3(n_nodes), dim3(SPLIT_TPB), 0, s, cands, feats, P,
                       nodes, cat_scratch, out, cat_out, cat_out_words, dev_n);
    return hipGetLastError();
}

// ======================================================================
// stable partition
// ======================================================================

__device__ __forceinline__ uint32_t find_req(const PartReqDev *reqs, uint32_t n, uint32_t chunk) {
    uint32_t lo = 0, hi = n;
    while (hi - lo > 1) {
        uint32_t mid = (lo + hi) >> 1;
        if (reqs[mid].chunk_begin <= chunk) lo = mid;
        else hi = mid;
    }
    return lo;
}

__device__ __forceinline__ uint32_t cell_of(const PartReqDev &R, uint32_t row) {
    const uint8_t *p = R.data + (size_t)row * R.stride + R.byte_off;
    return R.width == 1 ? (uint32_t)p[0] : (uint32_t) * reinterpret_cast<const uint16_t *>(p);
}

// The partition's go-left rule for a cell value of the request's feature.
__device__ __forceinline__ bool bin_goes_left(const PartReqDev &R, uint32_t bin,
                                              const uint64_t *cat_words) {
    if (bin == R.missing) return R.missing_left != 0;
    if (R.n_cat_words) {
        const uint32_t w = bin >> 6;
        const bool in = w < R.n_cat_words && ((cat_words[R.cat_off + w] >> (bin & 63)) & 1ull);
        return !in;
    }
    return bin < R.bin;
}

__device__ __forceinline__ bool goes_left(const PartReqDev &R, uint32_t row,
                                          const uint64_t *cat_words) {
    return bin_goes_left(R, cell_of(R, row), cat_words);
}

// Pass 1: direction flag per row and the left count of every chunk. A null
// row arena is the identity (rows in order).
__global__ __launch_bounds__(PART_TPB) void part_count_kernel(const PartReqDev *reqs,
                                                              uint32_t n_reqs,
                                                              const uint32_t *rows,
                                                              uint8_t *flags, uint32_t *counts,
                                                              const uint64_t *cat_words,
                                                              const uint32_t *dev) {
    constexpr int ROUNDS = PART_CHUNK / PART_TPB;
    __shared__ uint32_t wave_sum[PART_TPB / 64];
    const uint32_t chunk = blockIdx.x;
    if (dev && chunk >= dev[1]) return;
    const PartReqDev R = reqs[find_req(reqs, dev ? dev[0] : n_reqs, chunk)];
    const uint32_t c0 = (chunk - R.chunk_begin) * PART_CHUNK;
    const uint32_t c1 = min(c0 + PART_CHUNK, R.row_len);
    // All of the thread's row ids, then all of their cells, in flight at once.
    uint32_t row[ROUNDS], bin[ROUNDS];
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        const uint32_t i = c0 + r * PART_TPB + threadIdx.x;
        row[r] = i < c1 ? (rows ? rows[R.row_off + i] : R.row_off + i) : 0u;
    }
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        const uint32_t i = c0 + r * PART_TPB + threadIdx.x;
        bin[r] = i < c1 ? cell_of(R, row[r]) : 0u;
    }
    uint32_t cnt = 0;
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        const uint32_t i = c0 + r * PART_TPB + threadIdx.x;
        if (i < c1) {
            const bool gl = bin_goes_left(R, bin[r], cat_words);
            flags[R.row_off + i] = gl ? 1 : 0;
            cnt += gl;
        }
    }
    // wave reduction
    for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
    if ((threadIdx.x & 63) == 0) wave_sum[threadIdx.x >> 6] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int w = 0; w < PART_TPB / 64; w++) t += wave_sum[w];
        counts[R.count_base + (chunk - R.chunk_begin)] = t;
    }
}

// Pass 2: exclusive scan of the chunk counts (one workgroup) and the left
// total of every request.
__device__ void part_scan_body(const uint32_t *counts, uint32_t n_chunks, uint32_t *excl,
                               const PartReqDev *reqs, uint32_t n_reqs, uint32_t *totals,
                               const uint32_t *dev) {
    __shared__ uint32_t buf[32];
    if (dev) {
        n_reqs = dev[0];
        n_chunks = dev[1];
    }
    // Each thread a run of chunks: one block scan of the run sums.
    const uint32_t per = (n_chunks + 1023) / 1024;
    const uint32_t c0 = min(threadIdx.x * per, n_chunks), c1 = min(c0 + per, n_chunks);
    uint32_t sum = 0;
    for (uint32_t i = c0; i < c1; i++) sum += counts[i];
    uint32_t total;
    uint32_t run = block_scan_1024(sum, buf, total);
    for (uint32_t i = c0; i < c1; i++) {
        excl[i] = run;
        run += counts[i];
    }
    if (threadIdx.x == 0) excl[n_chunks] = total;
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < n_reqs; r += 1024)
        totals[r] = excl[reqs[r].chunk_begin + reqs[r].n_chunks] - excl[reqs[r].chunk_begin];
}

__global__ __launch_bounds__(1024) void part_scan_kernel(const uint32_t *counts, uint32_t n_chunks,
                                                         uint32_t *excl, const PartReqDev *reqs,
                                                         uint32_t n_reqs, uint32_t *totals,
                                                         const uint32_t *dev) {
    part_scan_body(counts, n_chunks, excl, reqs, n_reqs, totals, dev);
}

// part_scan_plan_kernel's scan when the chunks and requests fit LDS: the
// exclusive scan of the counts (a run of chunks a thread) kept in s_excl and
// written out for the scatter; the request totals from LDS into s_tot and
// totals.
__device__ __forceinline__ void part_scan_lds(const uint32_t *counts, uint32_t *excl,
                                              const PartReqDev *reqs, uint32_t *totals,
                                              uint32_t n_reqs, uint32_t n_chunks,
                                              uint32_t *s_excl, uint32_t *s_tot, uint32_t *buf) {
    uint32_t cb = 0, cn = 0;
    if (threadIdx.x < n_reqs) {
        cb = reqs[threadIdx.x].chunk_begin;
        cn = reqs[threadIdx.x].n_chunks;
    }
    // Exclusive scan of the counts (a run of chunks a thread), kept in LDS
    // and written out for the scatter; the request totals from LDS.
    const uint32_t per = (n_chunks + 1023) / 1024;
    const uint32_t c0 = min(threadIdx.x * per, n_chunks), c1 = min(c0 + per, n_chunks);
    uint32_t cnt[8];
    uint32_t sum = 0;
    if (per <= 8) {
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) {
            cnt[k] = c0 + k < c1 ? counts[c0 + k] : 0u;
            sum += cnt[k];
        }
    } else {
        for (uint32_t i = c0; i < c1; i++) sum += counts[i];
    }
    uint32_t total;
    uint32_t run = block_scan_1024(sum, buf, total);
    if (per <= 8) {
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) {
            if (c0 + k < c1) {
                s_excl[c0 + k] = run;
                excl[c0 + k] = run;
                run += cnt[k];
            }
        }
    } else {
        for (uint32_t i = c0; i < c1; i++) {
            s_excl[i] = run;
            excl[i] = run;
            run += counts[i];
        }
    }
    if (threadIdx.x == 0) {
        s_excl[n_chunks] = total;
        excl[n_chunks] = total;
    }
    __syncthreads();
    if (threadIdx.x < n_reqs) {
        const uint32_t t = s_excl[cb + cn] - s_excl[cb];
        s_tot[threadIdx.x] = t;
        totals[threadIdx.x] = t;
    }
    __syncthreads();
}

// Pass 2 of a device-grown level, fused with its plan: the scan, then (one
// workgroup, so the totals are visible after a barrier) the children plan of
// level_plan_kernel.
__global__ __launch_bounds__(1024) void part_scan_plan_kernel(
    const uint32_t *counts, uint32_t *excl, const PartReqDev *reqs, uint32_t *totals,
    const uint32_t *dev, const PairDev *pairs, ChunkRule rule, HistNodeDev *hn, SplitNodeDev *sn,
    uint32_t *spans, uint32_t *left_slot, uint32_t *chunk_rows_out, GrowDevOut D) {
    constexpr uint32_t LDS_CHUNKS = 8192;
    __shared__ uint32_t s_excl[LDS_CHUNKS + 1];
    __shared__ uint32_t s_tot[1024];
    __shared__ uint32_t buf[32];
    // Everything the scan and plan read that does not depend on the scan is
    // requested first: the counts, the state, the thread's request and pair.
    const uint32_t n_reqs = dev[0], n_chunks = dev[1];
    PlanPrefetch pre{};
    pre.valid = D.st != nullptr;
    if (pre.valid) {
        prefetch_state(pre, D.st);
        if (threadIdx.x < pre.n) pre.first = pairs[threadIdx.x];
    }
    // One inlined plan for both ways of scanning (the kernel's code is
    // fetched once a level: its size is latency).
    const bool big = n_chunks > LDS_CHUNKS || n_reqs > 1024;
    if (big) {
        part_scan_body(counts, 0u, excl, reqs, 0u, totals, dev);
        __syncthreads();
    } else {
        part_scan_lds(counts, excl, reqs, totals, n_reqs, n_chunks, s_excl, s_tot, buf);
    }
    level_plan_body(pairs, 0u, big ? totals : s_tot, rule, hn, sn, spans, left_slot,
                    chunk_rows_out, D, pre);
}


// Pass 3: stable scatter into the temporary arena. Rows of a chunk are taken
// in order, 256 at a time; a wave's lanes rank their rows with a ballot.
// Z.hist set: the workgroups also clear the histogram slots of the next
// level's accumulated nodes (those with several chunks, or all with force),
// as zero_nodes_kernel would, spread over the whole grid.
__global__ __launch_bounds__(PART_TPB) void part_scatter_kernel(const PartReqDev *reqs,
                                                                uint32_t n_reqs,
                                                                const uint32_t *rows,
                                                                const uint8_t *flags,
                                                                const uint32_t *excl,
                                                                const uint32_t *totals,
                                                                uint32_t *tmp,
                                                                const uint32_t *dev,
                                                                ZeroNodesDev Z) {
    if (Z.hist) {
        // The block's threads examine PART_TPB nodes at a time (one load
        // each) and list those to clear; only listed slots are visited.
        __shared__ uint32_t clr[PART_TPB];
        __shared__ uint32_t n_clr;
        const uint64_t W = Z.width * 2u;
        const uint32_t nn = *Z.dev_n;
        for (uint32_t e0 = 0; e0 < nn; e0 += PART_TPB) {
            if (threadIdx.x == 0) n_clr = 0;
            __syncthreads();
            const uint32_t e = e0 + threadIdx.x;
            if (e < nn) {
                const HistNodeDev N = Z.nodes[e];
                const bool clear = Z.group ? N.n_chunks > Z.group : (Z.force || N.n_chunks != 1);
                if (clear) clr[atomicAdd(&n_clr, 1u)] = N.slot;
            }
            __syncthreads();
            const uint32_t k = n_clr;
            for (uint32_t j = 0; j < k; j++) {
                int64_t *slot = Z.hist + (uint64_t)clr[j] * W;
                for (uint64_t i = (uint64_t)blockIdx.x * PART_TPB + threadIdx.x; i < W;
                     i += (uint64_t)gridDim.x * PART_TPB)
                    slot[i] = 0;
            }
            __syncthreads();
        }
    }
    const uint32_t chunk = blockIdx.x;
    if (dev && chunk >= dev[1]) return;
    const uint32_t ri = find_req(reqs, dev ? dev[0] : n_reqs, chunk);
    const PartReqDev R = reqs[ri];
    const uint32_t c0 = (chunk - R.chunk_begin) * PART_CHUNK;
    const uint32_t c1 = min(c0 + PART_CHUNK, R.row_len);
    const uint32_t left_base = excl[chunk] - excl[R.chunk_begin];
    const uint32_t total_left = totals[ri];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Every round's flags and row ids in flight at once, every round's
    // ballot counts in LDS behind one barrier.
    constexpr int ROUNDS = PART_CHUNK / PART_TPB;
    constexpr int WAVES = PART_TPB / 64;
    __shared__ uint32_t round_left[ROUNDS][WAVES];
    uint32_t row[ROUNDS], below[ROUNDS];
    uint32_t left_bits = 0;
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        const uint32_t i = c0 + r * PART_TPB + threadIdx.x;
        const bool valid = i < c1;
        row[r] = valid ? (rows ? rows[R.row_off + i] : R.row_off + i) : 0u;
        left_bits |= (valid && flags[R.row_off + i] ? 1u : 0u) << r;
    }
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        const uint64_t ball = __ballot((left_bits >> r) & 1u);
        below[r] = __popcll(ball & ((1ull << lane) - 1ull));
        if (lane == 0) round_left[r][wave] = __popcll(ball);
    }
    __syncthreads();
    uint32_t done_left = 0;  // lefts of earlier rounds in this chunk
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        uint32_t before = 0, in_round = 0;
        for (uint32_t w = 0; w < WAVES; w++) {
            if (w < wave) before += round_left[r][w];
            in_round += round_left[r][w];
        }
        const uint32_t i = c0 + r * PART_TPB + threadIdx.x;
        if (i < c1) {
            const uint32_t lrank = done_left + before + below[r];
            const uint32_t idx_in_chunk = i - c0;
            uint32_t dst;
            if ((left_bits >> r) & 1u) dst = R.row_off + left_base + lrank;
            else dst = R.row_off + total_left + (c0 - left_base) + (idx_in_chunk - lrank);
            tmp[dst] = row[r];
        }
        done_left += in_round;
    }
}

// A device-grown level's partition in one pass. Each workgroup takes one
// chunk of a split node's rows, finds every row's direction from the split
// feature's cell, and reserves places for its left rows at the front of the
// node's span and for its right rows at the back with one 64-bit atomic add
// on the node's cursor pair (left count in the low half, right count in the
// high half; zeroed by the level decision). Within a chunk the rows keep
// their order on each side; the chunks of a node take their places in the
// order their atomics land, so a child's rows are runs of ascending row ids
// in no fixed order. Everything computed from a node's rows is an integer sum
// (histograms, child sums) or per row (leaf assignment), so trees and margins
// do not depend on that order. The cursor's low half ends at the node's left
// count. A reservation past the node's span (cursors not zeroed) writes
// nothing and sets error bit 2.
__global__ __launch_bounds__(PART_TPB) void part_split_kernel(const PartReqDev *reqs,
                                                              const uint32_t *dev,
                                                              const uint32_t *rows_in,
                                                              uint32_t *rows_out,
                                                              unsigned long long *cursors,
                                                              const uint64_t *cat_words,
                                                              GrowState *st) {
    constexpr int ROUNDS = PART_CHUNK / PART_TPB;
    constexpr int WAVES = PART_TPB / 64;
    __shared__ uint32_t round_left[ROUNDS][WAVES];
    __shared__ uint32_t base_sh[2];
    const uint32_t chunk = blockIdx.x;
    if (chunk >= dev[1]) return;
    const uint32_t ri = find_req(reqs, dev[0], chunk);
    const PartReqDev R = reqs[ri];
    const uint32_t c0 = (chunk - R.chunk_begin) * PART_CHUNK;
    const uint32_t c1 = min(c0 + PART_CHUNK, R.row_len);
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // All of the thread's row ids, then all of their cells, in flight at once.
    uint32_t row[ROUNDS], bin[ROUNDS];
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        const uint32_t i = c0 + r * PART_TPB + threadIdx.x;
        row[r] = i < c1 ? (rows_in ? rows_in[R.row_off + i] : R.row_off + i) : 0u;
    }
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        const uint32_t i = c0 + r * PART_TPB + threadIdx.x;
        bin[r] = i < c1 ? cell_of(R, row[r]) : 0u;
    }
    uint32_t left_bits = 0, below[ROUNDS];
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        const uint32_t i = c0 + r * PART_TPB + threadIdx.x;
        const bool gl = i < c1 && bin_goes_left(R, bin[r], cat_words);
        left_bits |= (gl ? 1u : 0u) << r;
        const uint64_t ball = __ballot(gl);
        below[r] = __popcll(ball & ((1ull << lane) - 1ull));
        if (lane == 0) round_left[r][wave] = __popcll(ball);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t nl = 0;
        for (int r = 0; r < ROUNDS; r++)
            for (int w = 0; w < WAVES; w++) nl += round_left[r][w];
        const uint32_t nr = (c1 - c0) - nl;
        const unsigned long long old =
            atomicAdd(cursors + (uint64_t)ri * PART_CURSOR_STRIDE,
                      ((unsigned long long)nr << 32) | nl);
        const uint32_t lb = (uint32_t)old, rb = (uint32_t)(old >> 32);
        // Whatever order the chunks reserve in, the lefts and rights reserved
        // so far (this chunk's included) add up to at most the node's rows.
        const bool ok = (uint64_t)lb + nl + rb + nr <= R.row_len;
        base_sh[0] = lb;
        base_sh[1] = ok ? R.row_len - rb - nr : NO_SLOT;  // where this chunk's right rows start
        if (!ok) atomicOr(&st->error, 4u);
    }
    __syncthreads();
    const uint32_t lbase = base_sh[0], rstart = base_sh[1];
    if (rstart == NO_SLOT) return;
    uint32_t done_left = 0;  // lefts of earlier rounds in this chunk
#pragma unroll
    for (int r = 0; r < ROUNDS; r++) {
        uint32_t before = 0, in_round = 0;
        for (uint32_t w = 0; w < WAVES; w++) {
            if (w < wave) before += round_left[r][w];
            in_round += round_left[r][w];
        }
        const uint32_t i = c0 + r * PART_TPB + threadIdx.x;
        if (i < c1) {
            const uint32_t lrank = done_left + before + below[r];
            const uint32_t dst = ((left_bits >> r) & 1u)
                                     ? R.row_off + lbase + lrank
                                     : R.row_off + rstart + (i - c0 - lrank);
            rows_out[dst] = row[r];
        }
        done_left += in_round;
    }
}

// The children plan of a level partitioned by part_split_kernel: the left
// counts are the cursors' low halves.
__global__ __launch_bounds__(1024) void part_plan_kernel(
    const unsigned long long *cursors, uint32_t *totals, const PairDev *pairs, ChunkRule rule,
    HistNodeDev *hn, SplitNodeDev *sn, uint32_t *spans, uint32_t *left_slot,
    uint32_t *chunk_rows_out, GrowDevOut D) {
    __shared__ uint32_t s_tot[1024];
    PlanPrefetch pre{};
    pre.valid = true;
    prefetch_state(pre, D.st);
    if (threadIdx.x < pre.n) pre.first = pairs[threadIdx.x];
    // The left counts (low halves of the cursors) to the totals, read back
    // from LDS when they fit.
    const bool lds = pre.n <= 1024;
    for (uint32_t r = threadIdx.x; r < pre.n; r += 1024) {
        const uint32_t t = (uint32_t)cursors[(uint64_t)r * PART_CURSOR_STRIDE];
        totals[r] = t;
        if (lds) s_tot[r] = t;
    }
    __syncthreads();
    level_plan_body(pairs, 0u, lds ? s_tot : totals, rule, hn, sn, spans, left_slot,
                    chunk_rows_out, D, pre);
}

hipError_t launch_partition_split(const PartReqDev *reqs, const uint32_t *dev,
                                  uint32_t grid_chunks, const uint32_t *rows_in,
                                  uint32_t *rows_out, unsigned long long *cursors,
                                  uint32_t *totals, const uint64_t *cat_words,
                                  const PairDev *pairs, ChunkRule rule, HistNodeDev *hn,
                                  SplitNodeDev *sn, uint32_t *spans, uint32_t *left_slot,
                                  uint32_t *chunk_rows, const GrowDevOut &D, hipStream_t s) {
    if (grid_chunks == 0 || !D.st) return hipErrorInvalidValue;
    hipLaunchKernelGGL(part_split_kernel, dim3(grid_chunks), dim3(PART_TPB), 0, s, reqs, dev,
                       rows_in, rows_out, cursors, cat_words, D.st);
    hipLaunchKernelGGL(part_plan_kernel, dim3(1), dim3(1024), 0, s, cursors, totals, pairs, rule,
                       hn, sn, spans, left_slot, chunk_rows, D);
    return hipGetLastError();
}

__global__ __launch_bounds__(PART_TPB) void part_copy_kernel(const PartReqDev *reqs,
                                                             uint32_t n_reqs, const uint32_t *tmp,
                                                             uint32_t *rows, const uint32_t *dev) {
    const uint32_t chunk = blockIdx.x;
    if (dev && chunk >= dev[1]) return;
    const PartReqDev R = reqs[find_req(reqs, dev ? dev[0] : n_reqs, chunk)];
    const uint32_t c0 = (chunk - R.chunk_begin) * PART_CHUNK;
    const uint32_t c1 = min(c0 + PART_CHUNK, R.row_len);
    for (uint32_t i = c0 + threadIdx.x; i < c1; i += PART_TPB)
        rows[R.row_off + i] = tmp[R.row_off + i];
}

hipError_t launch_partition_count(const PartReqDev *reqs, uint32_t n_reqs, uint32_t n_chunks,
                                  const uint32_t *rows, uint8_t *flags, uint32_t *counts,
                                  const uint64_t *cat_words, hipStream_t s) {
    if (n_chunks == 0) return hipSuccess;
    hipLaunchKernelGGL(part_count_kernel, dim3(n_chunks), dim3(PART_TPB), 0, s, reqs, n_reqs, rows,
                       flags, counts, cat_words, nullptr);
    return hipGetLastError();
}

hipError_t launch_partition_level(const PartReqDev *reqs, const uint32_t *dev, uint32_t grid_chunks,
                                  const uint32_t *rows_in, uint32_t *rows_out, uint8_t *flags,
                                  uint32_t *counts, uint32_t *excl, uint32_t *totals,
                                  const uint64_t *cat_words, const PairDev *pairs, ChunkRule rule,
                                  HistNodeDev *hn, SplitNodeDev *sn, uint32_t *spans,
                                  uint32_t *left_slot, uint32_t *chunk_rows, const GrowDevOut &D,
                                  const ZeroNodesDev &Z, hipStream_t s) {
    if (grid_chunks == 0) return hipSuccess;
    hipLaunchKernelGGL(part_count_kernel, dim3(grid_chunks), dim3(PART_TPB), 0, s, reqs, 0u,
                       rows_in, flags, counts, cat_words, dev);
    hipLaunchKernelGGL(part_scan_plan_kernel, dim3(1), dim3(1024), 0, s, counts, excl, reqs, totals,
                       dev, pairs, rule, hn, sn, spans, left_slot, chunk_rows, D);
    hipLaunchKernelGGL(part_scatter_kernel, dim3(grid_chunks), dim3(PART_TPB), 0, s, reqs, 0u,
                       rows_in, flags, excl, totals, rows_out, dev, Z);
    return hipGetLastError();
}

hipError_t launch_partition_finish(const PartReqDev *reqs, uint32_t n_reqs, uint32_t n_chunks,
                                   uint32_t *rows, uint32_t *tmp, const uint8_t *flags,
                                   const uint32_t *counts, uint32_t *excl, uint32_t *totals,
                                   hipStream_t s) {
    if (n_chunks == 0) return hipSuccess;
    hipLaunchKernelGGL(part_scan_kernel, dim3(1), dim3(1024), 0, s, counts, n_chunks, excl, reqs,
                       n_reqs, totals, nullptr);
    hipLaunchKernelGGL(part_scatter_kernel, dim3(n_chunks), dim3(PART_TPB), 0, s, reqs, n_reqs,
                       rows, flags, excl, totals, tmp, nullptr, ZeroNodesDev{});
    hipLaunchKernelGGL(part_copy_kernel, dim3(n_chunks), dim3(PART_TPB), 0, s, reqs, n_reqs, tmp,
                       rows, nullptr);
    return hipGetLastError();
}

// ======================================================================
// leaves, row arena, quantisation, tile packing
// ======================================================================

// SplitMix64 finaliser (subsample::mix, src/data/subsample.rs).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t rotl64(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }

// IDB == 0: delta[row] = leaf value; IDB == 1 / 2: ids[row] = leaf position
// as u8 / u16 (the margins are then updated in row order by apply_leaves).
template <int IDB>
__global__ __launch_bounds__(PART_TPB) void leaf_kernel(const LeafDev *leaves, uint32_t n,
                                                        const uint32_t *rows,
                                                        const uint32_t *rows_alt, float *delta,
                                                        void *ids, const uint32_t *dev) {
    const uint32_t chunk = blockIdx.x;
    if (dev) {  // a device-grown tree: leaf count and chunks on the device
        if (chunk >= dev[1]) return;
        n = dev[0];
    }
    uint32_t lo = 0, hi = n;
    while (hi - lo > 1) {
        uint32_t mid = (lo + hi) >> 1;
        if (leaves[mid].chunk_begin <= chunk) lo = mid;
        else hi = mid;
    }
    const LeafDev L = leaves[lo];
    const uint32_t c0 = (chunk - L.chunk_begin) * PART_CHUNK;
    const uint32_t c1 = min(c0 + PART_CHUNK, L.row_len);
    const uint32_t *rr = L.arena ? rows_alt : rows;
    for (uint32_t i = c0 + threadIdx.x; i < c1; i += PART_TPB) {
        const uint32_t r = rr[L.row_off + i];
        if (IDB == 0) delta[r] = L.value;
        if (IDB == 1) static_cast<uint8_t *>(ids)[r] = (uint8_t)L.id;
        if (IDB == 2) static_cast<uint16_t *>(ids)[r] = (uint16_t)L.id;
    }
}

// margin[row] += values[ids[row]] in row order: the same f32 addition as the
// host's pred += delta.
template <int IDB>
__global__ __launch_bounds__(256) void apply_leaves_kernel(const void *ids, const float *values,
                                                           uint64_t n, float *margin) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t id = IDB == 1 ? (uint32_t) static_cast<const uint8_t *>(ids)[i]
                                     : (uint32_t) static_cast<const uint16_t *>(ids)[i];
        margin[i] = margin[i] + values[id];
    }
}

hipError_t launch_assign_leaves(const LeafDev *leaves, uint32_t n_leaves, uint32_t n_chunks,
                                const uint32_t *rows, const uint32_t *rows_alt, float *delta,
                                void *ids, int id_bytes, const uint32_t *dev, hipStream_t s) {
    if (n_chunks == 0) return hipSuccess;
    if (id_bytes == 1)
        hipLaunchKernelGGL(leaf_kernel<1>, dim3(n_chunks), dim3(PART_TPB), 0, s, leaves, n_leaves,
                           rows, rows_alt, delta, ids, dev);
    else if (id_bytes == 2)
        hipLaunchKernelGGL(leaf_kernel<2>, dim3(n_chunks), dim3(PART_TPB), 0, s, leaves, n_leaves,
                           rows, rows_alt, delta, ids, dev);
    else
        hipLaunchKernelGGL(leaf_kernel<0>, dim3(n_chunks), dim3(PART_TPB), 0, s, leaves, n_leaves,
                           rows, rows_alt, delta, ids, dev);
    return hipGetLastError();
}

hipError_t launch_apply_leaves(const void *ids, int id_bytes, const float *values, uint64_t n,
                               float *margin, hipStream_t s) {
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((n + 255) / 256, 8192);
    if (blocks == 0) return hipSuccess;
    if (id_bytes == 1)
        hipLaunchKernelGGL(apply_leaves_kernel<1>, dim3(blocks), dim3(256), 0, s, ids, values, n,
                           margin);
    else
        hipLaunchKernelGGL(apply_leaves_kernel<2>, dim3(blocks), dim3(256), 0, s, ids, values, n,
                           margin);
    return hipGetLastError();
}

// Objective::gradient (src/training/objective.rs:499-530), restated in f32
// with the host's operation order; compiled without FMA contraction, so the
// pairs equal the host's bit for bit. mode 0: squared error from the margin;
// 1: logistic from the host's sigmoid in src; 2: logistic from the margin
// with the device sigmoid (bit-identical to the host's libm); 3: logistic
// from the margin with the hardware exponential (gpu_math="fast", the
// reference's apply_delta_and_gradient, src/backend/cuda/histogram.cu:
// 673-783: deterministic, not bit-equal to the host).
__device__ __forceinline__ float fast_sigmoid(float m) { return 1.0f / (1.0f + __expf(-m)); }

__device__ __forceinline__ float objective_source(int mode, float v) {
    return mode == 2 ? fb_sigmoid(v) : mode == 3 ? fast_sigmoid(v) : v;
}

// One row's weighted pair. Modes 0-3: squared error (0) or logistic from the
// source value (1: host sigmoids, 2: the exact device sigmoid, 3: the fast
// one); g = v - y, h = max(v (1 - v), 1e-16) (1 for squared error), both
// times the weight. Modes 4/5: softmax class cls from the round's row
// statistics st = (wmax, wsum) (Objective::softmax_gradients,
// src/training/objective.rs:1175-1219; 4: glibc's expf restated, 5: the
// hardware exp): p = exp(m - wmax) / wsum, h = max(2 p (1 - p) w, 1e-16),
// g = (p - [y == cls]) w. Mode 6: reg:quantileerror under the round's
// (scale S, alpha) in stats[0] (Objective::quantile_gradient,
// objective.rs:1142-1160): x = (m - y) / (0.04 S),
// g = S/2 (tanh x + 1 - 2 alpha), h = 12.5 max(tanh x / x, 3e-4) (1 at
// x = 0), both times the weight, (0, 0) unless S > 0; tanh is glibc's tanhf
// restated, the host's values bit for bit.
__device__ __forceinline__ void row_pair(int mode, float s, float y, bool has_w, float w,
                                         const float2 *stats, uint32_t cls, uint64_t i, float &g,
                                         float &h) {
    if (mode == 6) {
        const float2 q = stats[0];
        const float scale = q.x, alpha = q.y;
        if (!(scale > 0.0f)) {
            g = h = 0.0f;
            return;
        }
        const float x = (s - y) / (0.04f * scale);
        const float t = fb_tanhf(x);
        float ratio = x == 0.0f ? 1.0f : t / x;
        ratio = fmaxf(ratio, 3.0e-4f);
        g = 0.5f * scale * (t + 1.0f - 2.0f * alpha);
        h = 0.5f / 0.04f * ratio;
        if (has_w) {
            g = g * w;
            h = h * w;
        }
        return;
    }
    if (mode >= 4) {
        const float2 st = stats[i];
        const float e = mode == 4 ? fb_expf(s - st.x) : __expf(s - st.x);
        float p = e / st.y;
        const float wt = has_w ? w : 1.0f;
        h = fmaxf(2.0f * p * (1.0f - p) * wt, 1e-16f);
        if (y == (float)cls) p = p - 1.0f;
        g = p * wt;
        return;
    }
    const float v = objective_source(mode, s);
    g = v - y;
    h = mode != 0 ? fmaxf(v * (1.0f - v), 1e-16f) : 1.0f;
    if (has_w) {
        g = g * w;
        h = h * w;
    }
}

// softmax_row_stats (src/backend/cuda/histogram.cu:786-835; the row loop of
// Objective::softmax_gradients): per row, the largest of the K class margins
// (from the smallest normal float up) and the sum over classes, in class
// order and in double, of exp(m - wmax); the sum is kept as a float, the
// divisor every class uses.
__global__ __launch_bounds__(256) void softmax_stats_kernel(const float *margin, uint32_t K,
                                                            uint64_t n, int fast, float2 *stats) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        float wmax = 1.17549435e-38f;
        for (uint32_t k = 0; k < K; k++) wmax = fmaxf(margin[(uint64_t)k * n + i], wmax);
        double wsum = 0.0;
        for (uint32_t k = 0; k < K; k++) {
            const float d = margin[(uint64_t)k * n + i] - wmax;
            wsum += (double)(fast ? __expf(d) : fb_expf(d));
        }
        stats[i] = make_float2(wmax, (float)wsum);
    }
}

// The terms of the quantile scale (Objective::quantile_scale,
// objective.rs:1115-1137): per row the f32 value w * sqrtf|m - y| (sqrtf|m - y|
// without weights), which the host sums in row order in double.
__global__ __launch_bounds__(256) void quantile_terms_kernel(const float *margin, const float *y,
                                                             const float *w, uint64_t n,
                                                             float *out) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const float r = sqrtf(fabsf(margin[i] - y[i]));
        out[i] = w ? w[i] * r : r;
    }
}

hipError_t launch_quantile_terms(const float *margin, const float *y, const float *w, uint64_t n,
                                 float *out, hipStream_t s) {
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((n + 255) / 256, 8192);
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(quantile_terms_kernel, dim3(blocks), dim3(256), 0, s, margin, y, w, n, out);
    return hipGetLastError();
}

__global__ void quantile_set_kernel(float2 *slot, float scale, float alpha) {
    if (threadIdx.x == 0) slot[0] = make_float2(scale, alpha);
}

hipError_t launch_quantile_set(float2 *slot, float scale, float alpha, hipStream_t s) {
    hipLaunchKernelGGL(quantile_set_kernel, dim3(1), dim3(64), 0, s, slot, scale, alpha);
    return hipGetLastError();
}

// gpu_math="fast": the scale on the device in a fixed order (the reference's
// quantile_apply_delta_partials / quantile_reduce_scale,
// src/backend/cuda/histogram.cu:907-1010): each of QUANTILE_BLOCKS x 256
// threads sums its grid-stride rows in double, a fixed tree sums each
// block, and one workgroup sums the block partials the same way, so every
// run gives the same scale (not the host's serial sum).
constexpr uint32_t QUANTILE_BLOCKS = 256;

__global__ __launch_bounds__(256) void quantile_partials_kernel(const float *margin,
                                                                const float *y, const float *w,
                                                                uint64_t n, double *partials) {
    __shared__ double rs[256], rw[256];
    double stat = 0.0, sum_w = 0.0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const float r = sqrtf(fabsf(margin[i] - y[i]));
        if (w) {
            stat += (double)(w[i] * r);
            sum_w += (double)w[i];
        } else {
            stat += (double)r;
        }
    }
    rs[threadIdx.x] = stat;
    rw[threadIdx.x] = sum_w;
    __syncthreads();
    for (uint32_t k = 128; k > 0; k >>= 1) {
        if (threadIdx.x < k) {
            rs[threadIdx.x] += rs[threadIdx.x + k];
            rw[threadIdx.x] += rw[threadIdx.x + k];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        partials[2 * blockIdx.x] = rs[0];
        partials[2 * blockIdx.x + 1] = rw[0];
    }
}

__global__ __launch_bounds__(256) void quantile_reduce_kernel(const double *partials,
                                                              uint64_t n, int weighted,
                                                              float alpha, float2 *slot) {
    __shared__ double rs[256], rw[256];
    rs[threadIdx.x] = partials[2 * threadIdx.x];
    rw[threadIdx.x] = partials[2 * threadIdx.x + 1];
    __syncthreads();
    for (uint32_t k = 128; k > 0; k >>= 1) {
        if (threadIdx.x < k) {
            rs[threadIdx.x] += rs[threadIdx.x + k];
            rw[threadIdx.x] += rw[threadIdx.x + k];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const double total_w = weighted ? rw[0] : (double)n;
        float scale = 0.0f;
        if (!(fabs(total_w) < 1e-6)) {
            const double root_mean = rs[0] / total_w;
            scale = (float)(root_mean * root_mean);
        }
        slot[0] = make_float2(scale, alpha);
    }
}

hipError_t launch_quantile_scale_fast(const float *margin, const float *y, const float *w,
                                      uint64_t n, float alpha, double *partials, float2 *slot,
                                      hipStream_t s) {
    hipLaunchKernelGGL(quantile_partials_kernel, dim3(QUANTILE_BLOCKS), dim3(256), 0, s, margin,
                       y, w, n, partials);
    hipLaunchKernelGGL(quantile_reduce_kernel, dim3(1), dim3(QUANTILE_BLOCKS), 0, s, partials, n,
                       w ? 1 : 0, alpha, slot);
    return hipGetLastError();
}

// A grown tree's result into pinned host memory from the stream's own queue
// (a copy-engine transfer makes the compute queue wait for a handoff between
// engines, measured at 50-75 us a tree): the state, then the used nodes,
// category words and leaf values at their offsets in `out` (a device view of
// the host buffer). Counts come from the state and are clamped to the
// capacities.
__device__ __forceinline__ void copy_words(const void *src, void *dst, uint64_t bytes,
                                           uint64_t t, uint64_t T) {
    const uint32_t *s = static_cast<const uint32_t *>(src);
    uint32_t *d = static_cast<uint32_t *>(dst);
    for (uint64_t i = t; i < bytes / 4; i += T) d[i] = s[i];
}

__global__ __launch_bounds__(256) void tree_out_kernel(const GrowState *st, const TreeNodeDev *tree,
                                                       uint32_t tree_cap, const uint64_t *cats,
                                                       uint32_t cat_cap, const float *vals,
                                                       uint32_t leaf_cap, uint8_t *out,
                                                       uint64_t o_tree, uint64_t o_cats,
                                                       uint64_t o_vals) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t T = (uint64_t)gridDim.x * blockDim.x;
    const uint32_t nt = min(st->tree_size, tree_cap);
    const uint32_t nl = min(st->n_leaves, leaf_cap);
    const uint32_t nc = cats ? min(st->tree_cat_words, cat_cap) : 0u;
    copy_words(st, out, sizeof(GrowState), t, T);
    copy_words(tree, out + o_tree, (uint64_t)nt * sizeof(TreeNodeDev), t, T);
    if (nc) copy_words(cats, out + o_cats, (uint64_t)nc * 8, t, T);
    copy_words(vals, out + o_vals, (uint64_t)nl * 4, t, T);
    __threadfence_system();
}

hipError_t launch_tree_out(const GrowState *st, const TreeNodeDev *tree, uint32_t tree_cap,
                           const uint64_t *cats, uint32_t cat_cap, const float *vals,
                           uint32_t leaf_cap, uint8_t *out, uint64_t o_tree, uint64_t o_cats,
                           uint64_t o_vals, hipStream_t s) {
    hipLaunchKernelGGL(tree_out_kernel, dim3(8), dim3(256), 0, s, st, tree, tree_cap, cats,
                       cat_cap, vals, leaf_cap, out, o_tree, o_cats, o_vals);
    return hipGetLastError();
}

// bytes from src (a device view of coherent pinned host memory) to dst, in
// the stream (no copy engine): four-byte words, then the tail.
__global__ __launch_bounds__(256) void copy_bytes_kernel(uint8_t *dst, const uint8_t *src,
                                                         uint64_t bytes) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t T = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t words = bytes / 4;
    if ((((uintptr_t)dst | (uintptr_t)src) & 3u) == 0) {
        const uint32_t *s = reinterpret_cast<const uint32_t *>(src);
        uint32_t *d = reinterpret_cast<uint32_t *>(dst);
        for (uint64_t i = t; i < words; i += T) d[i] = s[i];
        for (uint64_t i = 4 * words + t; i < bytes; i += T) dst[i] = src[i];
    } else {
        for (uint64_t i = t; i < bytes; i += T) dst[i] = src[i];
    }
}

hipError_t launch_copy_bytes(void *dst, const void *src, uint64_t bytes, hipStream_t s) {
    if (bytes == 0) return hipSuccess;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((bytes / 4 + 255) / 256 + 1, 64);
    hipLaunchKernelGGL(copy_bytes_kernel, dim3(blocks), dim3(256), 0, s,
                       static_cast<uint8_t *>(dst), static_cast<const uint8_t *>(src), bytes);
    return hipGetLastError();
}

hipError_t launch_softmax_stats(const float *margin, uint32_t K, uint64_t n, int fast,
                                float2 *stats, hipStream_t s) {
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((n + 255) / 256, 8192);
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(softmax_stats_kernel, dim3(blocks), dim3(256), 0, s, margin, K, n, fast,
                       stats);
    return hipGetLastError();
}
__device__ __forceinline__ bool row_selected(uint64_t row, uint64_t th, uint64_t seed,
                                             uint64_t tree);
__device__ __forceinline__ double finite_abs(float v);
__device__ void block_max2(double mg, double mh, double *block_max);

__device__ __forceinline__ int64_t sat_i64(double x);
__device__ void block_sum2(uint64_t ag, uint64_t ah, int64_t *block_sum);

// block_max set: rows outside the round's subsample get a zero pair, and
// each block's max |g|, max |h| goes to block_max (the bounds pass fused in).
// g2n set: the f32 pairs go there. spec set: the fixed-point pairs under the
// scales in spec (the previous round's) go to fixed (when set), with the block sums; the bounds
// pass then tells whether those were this round's scales
// (gradient_fixup_kernel redoes the pairs when not). The same grid and
// operations as without spec, so each row's g and h are the same floats.
// Calls f with std::integral_constant<int, mode> for the gradient modes 0-6.
template <class F>
hipError_t with_mode(int mode, F &&f) {
    switch (mode) {
        case 0: return f(std::integral_constant<int, 0>{});
        case 1: return f(std::integral_constant<int, 1>{});
        case 2: return f(std::integral_constant<int, 2>{});
        case 3: return f(std::integral_constant<int, 3>{});
        case 4: return f(std::integral_constant<int, 4>{});
        case 5: return f(std::integral_constant<int, 5>{});
        case 6: return f(std::integral_constant<int, 6>{});
        default: return hipErrorInvalidValue;
    }
}

// The objective mode is a template argument, so each objective's kernel
// holds only its own arithmetic (and registers).
template <int MODE>
__global__ __launch_bounds__(256) void gradient_kernel(const float *src, const float *y,
                                                       const float *w, uint64_t n,
                                                       float *g2n, uint64_t th, uint64_t seed,
                                                       uint64_t tree, double *block_max,
                                                       const ScalesDev *spec, int64_t *fixed,
                                                       int64_t *block_sum, const float2 *stats,
                                                       uint32_t cls) {
    // Four rows a thread per step (loads of all four first).
    constexpr int U = 4;
    double mg = 0.0, mh = 0.0;
    uint64_t ag = 0, ah = 0;
    double sg = 0.0, sh = 0.0;
    if (spec) {
        sg = spec->scale[0];
        sh = spec->scale[1];
    }
    const uint64_t S = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t base = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; base < n;
         base += U * S) {
        float sv[U], yv[U], wv[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint64_t i = base + u * S;
            const bool ok = i < n;
            sv[u] = ok ? src[i] : 0.0f;
            yv[u] = ok ? y[i] : 0.0f;
            wv[u] = (ok && w) ? w[i] : 1.0f;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint64_t i = base + u * S;
            if (i >= n) continue;
            float g, h;
            row_pair(MODE, sv[u], yv[u], w != nullptr, wv[u], stats, cls, i, g, h);
            if (block_max) {
                if (!row_selected(i, th, seed, tree)) g = h = 0.0f;
                mg = fmax(mg, finite_abs(g));
                mh = fmax(mh, finite_abs(h));
            }
            if (spec) {
                const int64_t qg = sat_i64(round((double)g * sg));
                const int64_t qh = sat_i64(round((double)h * sh));
                if (fixed) reinterpret_cast<longlong2 *>(fixed)[i] = make_longlong2(qg, qh);
                ag += (uint64_t)qg;
                ah += (uint64_t)qh;
            }
            if (g2n) reinterpret_cast<float2 *>(g2n)[i] = make_float2(g, h);
        }
    }
    if (block_max) block_max2(mg, mh, block_max);
    if (spec) block_sum2(ag, ah, block_sum);
}

// After a speculative gradient pass: when the bounds gave other scales than
// the ones the pass used, the pairs and block sums are computed again (the
// same gradient) under the right scales; otherwise every block leaves at once.
template <int MODE>
__global__ __launch_bounds__(256) void gradient_fixup_kernel(const float *src, const float *y,
                                                             const float *w, uint64_t n,
                                                             uint64_t th, uint64_t seed,
                                                             uint64_t tree,
                                                             const ScalesDev *scales,
                                                             int64_t *fixed, int64_t *block_sum,
                                                             const float2 *stats, uint32_t cls) {
    if (!scales->spec_miss) return;  // uniform
    const double sg = scales->scale[0], sh = scales->scale[1];
    uint64_t ag = 0, ah = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        float g, h;
        row_pair(MODE, src[i], y[i], w != nullptr, w ? w[i] : 1.0f, stats, cls, i, g, h);
        if (!row_selected(i, th, seed, tree)) g = h = 0.0f;
        const int64_t qg = sat_i64(round((double)g * sg));
        const int64_t qh = sat_i64(round((double)h * sh));
        if (fixed) reinterpret_cast<longlong2 *>(fixed)[i] = make_longlong2(qg, qh);
        ag += (uint64_t)qg;
        ah += (uint64_t)qh;
    }
    block_sum2(ag, ah, block_sum);
}

__global__ void reduce_max_kernel(const double *block_max, uint32_t n, double *out,
                                  uint64_t n_rows, ScalesDev *scales);

hipError_t launch_gradient_spec(const float *src, const float *y, const float *w, uint64_t n,
                                int mode, uint64_t th, uint64_t seed, uint64_t tree,
                                double *block_max, uint32_t n_blocks, ScalesDev *scales,
                                int64_t *fixed, int64_t *block_sum, float *g2n, hipStream_t s,
                                const float2 *stats, uint32_t cls) {
    if (n_blocks == 0) return hipSuccess;
    return with_mode(mode, [&](auto M) {
        constexpr int MODE = decltype(M)::value;
        hipLaunchKernelGGL(gradient_kernel<MODE>, dim3(n_blocks), dim3(256), 0, s, src, y, w, n,
                           g2n, th, seed, tree, block_max, scales, fixed, block_sum, stats, cls);
        hipLaunchKernelGGL(reduce_max_kernel, dim3(1), dim3(1024), 0, s, block_max, n_blocks,
                           block_max + 2 * n_blocks, n, scales);
        hipLaunchKernelGGL(gradient_fixup_kernel<MODE>, dim3(n_blocks), dim3(256), 0, s, src, y,
                           w, n, th, seed, tree, scales, fixed, block_sum, stats, cls);
        return hipGetLastError();
    });
}

hipError_t launch_gradient(const float *src, const float *y, const float *w, uint64_t n, int mode,
                           float *g2n, uint64_t th, uint64_t seed, uint64_t tree,
                           double *block_max, uint32_t n_blocks, hipStream_t s,
                           const float2 *stats, uint32_t cls) {
    const uint32_t blocks =
        block_max ? n_blocks : (uint32_t)std::min<uint64_t>((n + 255) / 256, 8192);
    if (blocks == 0) return hipSuccess;
    return with_mode(mode, [&](auto M) {
        constexpr int MODE = decltype(M)::value;
        hipLaunchKernelGGL(gradient_kernel<MODE>, dim3(blocks), dim3(256), 0, s, src, y, w, n,
                           g2n, th, seed, tree, block_max, nullptr, nullptr, nullptr, stats, cls);
        return hipGetLastError();
    });
}

__global__ __launch_bounds__(256) void sigmoid_kernel(const float *in, uint64_t n, float *out) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = fb_sigmoid(in[i]);
}

hipError_t launch_sigmoid(const float *in, uint64_t n, float *out, hipStream_t s) {
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((n + 255) / 256, 8192);
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(sigmoid_kernel, dim3(blocks), dim3(256), 0, s, in, n, out);
    return hipGetLastError();
}

// Sum over bit patterns u in [begin, end) of mix64(u ^ bits(f(u)) << 32)
// (NaN outputs canonicalised), wrapping: a fingerprint of the device sigmoid
// (TANH false) or tanhf (TANH true) over every float input, compared with
// the host libm's.
template <bool TANH>
__global__ __launch_bounds__(256) void sigmoid_checksum_kernel(uint64_t begin, uint64_t end,
                                                               unsigned long long *out) {
    uint64_t acc = 0;
    for (uint64_t u = begin + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; u < end;
         u += (uint64_t)gridDim.x * blockDim.x) {
        const float x = __builtin_bit_cast(float, (uint32_t)u);
        const float s = TANH ? fb_tanhf(x) : fb_sigmoid(x);
        const uint32_t b = s != s ? 0x7fc00000u : __builtin_bit_cast(uint32_t, s);
        acc += mix64(u ^ ((uint64_t)b << 32));
    }
    __shared__ uint64_t sm[256];
    sm[threadIdx.x] = acc;
    __syncthreads();
    for (uint32_t k = 128; k > 0; k >>= 1) {
        if (threadIdx.x < k) sm[threadIdx.x] += sm[threadIdx.x + k];
        __syncthreads();
    }
    if (threadIdx.x == 0) global_add_u64(out, sm[0]);
}

hipError_t launch_sigmoid_checksum(uint64_t begin, uint64_t end, unsigned long long *out,
                                   hipStream_t s, bool tanh) {
    if (end <= begin) return hipSuccess;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((end - begin + 255) / 256, 65536);
    if (tanh)
        hipLaunchKernelGGL(sigmoid_checksum_kernel<true>, dim3(blocks), dim3(256), 0, s, begin,
                           end, out);
    else
        hipLaunchKernelGGL(sigmoid_checksum_kernel<false>, dim3(blocks), dim3(256), 0, s, begin,
                           end, out);
    return hipGetLastError();
}

__global__ void fill_f32_kernel(float *p, float v, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

hipError_t launch_fill_f32(float *p, float v, uint64_t n, hipStream_t s) {
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((n + 255) / 256, 4096);
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_f32_kernel, dim3(blocks), dim3(256), 0, s, p, v, n);
    return hipGetLastError();
}

__global__ void init_rows_kernel(uint32_t *rows, float *delta, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        rows[i] = (uint32_t)i;
        if (delta) delta[i] = 0.0f;
    }
}

hipError_t launch_init_rows(uint32_t *rows, float *delta, uint64_t n, hipStream_t s) {
    uint32_t blocks = (uint32_t)std::min<uint64_t>((n + 255) / 256, 4096);
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(init_rows_kernel, dim3(blocks), dim3(256), 0, s, rows, delta, n);
    return hipGetLastError();
}


// subsample::row_selected (src/data/subsample.rs).
__device__ __forceinline__ bool row_selected(uint64_t row, uint64_t th, uint64_t seed,
                                             uint64_t tree) {
    if (th == ~0ull) return true;
    const uint64_t hsh = mix64(seed ^ rotl64(tree * 0x9E3779B97F4A7C15ull, 23) ^
                               (row * 0xD6E8FEB86659FD93ull));
    return (hsh >> 11) < th;
}

__device__ __forceinline__ double finite_abs(float v) {
    return isfinite(v) ? fabs((double)v) : (double)INFINITY;
}

// Block maxima of the two bounds (256 threads) into block_max[2 * block]:
// shuffles within each wave, then the four wave results.
__device__ void block_max2(double mg, double mh, double *block_max) {
    __shared__ double sm[2][4];
    for (int off = 32; off > 0; off >>= 1) {
        mg = fmax(mg, __shfl_xor(mg, off, 64));
        mh = fmax(mh, __shfl_xor(mh, off, 64));
    }
    if ((threadIdx.x & 63) == 0) {
        sm[0][threadIdx.x >> 6] = mg;
        sm[1][threadIdx.x >> 6] = mh;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        block_max[2 * blockIdx.x] = fmax(fmax(sm[0][0], sm[0][1]), fmax(sm[0][2], sm[0][3]));
        block_max[2 * blockIdx.x + 1] = fmax(fmax(sm[1][0], sm[1][1]), fmax(sm[1][2], sm[1][3]));
    }
}

// Wrapping block sums of the two components (256 threads) into
// block_sum[2 * block].
__device__ void block_sum2(uint64_t ag, uint64_t ah, int64_t *block_sum) {
    __shared__ int64_t sm[2][4];
    for (int off = 32; off > 0; off >>= 1) {
        ag += (uint64_t)__shfl_xor((long long)ag, off, 64);
        ah += (uint64_t)__shfl_xor((long long)ah, off, 64);
    }
    if ((threadIdx.x & 63) == 0) {
        sm[0][threadIdx.x >> 6] = (int64_t)ag;
        sm[1][threadIdx.x >> 6] = (int64_t)ah;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        block_sum[2 * blockIdx.x] = wadd(wadd(sm[0][0], sm[0][1]), wadd(sm[0][2], sm[0][3]));
        block_sum[2 * blockIdx.x + 1] = wadd(wadd(sm[1][0], sm[1][1]), wadd(sm[1][2], sm[1][3]));
    }
}

// floor(log2(x)) for a positive, finite, normal x as the floor of a correctly
// rounded log2(x) gives it (the host's `log2(raw).floor()`): the exact floor,
// except when log2(x) lies less than half a double spacing below an integer,
// where the rounded logarithm is that integer.
__device__ int floor_rounded_log2(double x) {
    int e;
    const double f = frexp(x, &e);  // x = f * 2^e, f in [0.5, 1)
    if (f == 0.5) return e - 1;     // a power of two
    if (e == 0) return -1;          // log2(x) in (-1, 0), never rounded to 0
    // log2(x) = e - eps, eps = -log2(f) in (0, 1); f - 1 is exact.
    const double eps = -log1p(f - 1.0) / 0.69314718055994530942;
    const int ae = e > 0 ? e : -e;
    const int a = 31 - __clz(ae);  // |e| in [2^a, 2^(a+1))
    // Spacing of the doubles next to e on the side of e - eps.
    const double spacing =
        (e > 0 && (ae & (ae - 1)) == 0) ? ldexp(1.0, a - 53) : ldexp(1.0, a - 52);
    return eps < 0.5 * spacing ? e : e - 1;
}

// GradQuantizer::try_from_bounds (src/types.rs:288-303): a power-of-two
// scale per component with max_abs * n_rows * scale below 2^62.
__device__ double scale_from_bound(double m, uint64_t n_rows) {
    if (!(m > 0.0) || !isfinite(m)) return 1.0;
    const double budget = 4611686018427387904.0 / (double)(n_rows ? n_rows : 1);
    const double raw = budget / m;
    if (!isfinite(raw) || !(raw > 0.0)) return 1.0;
    int l = floor_rounded_log2(raw);
    l = l > 1000 ? 1000 : (l < -1000 ? -1000 : l);
    return ldexp(1.0, l);
}

// Masks sampled-out rows (in place) and reduces max |g|, max |h| per block.
__global__ __launch_bounds__(256) void gpair_maxabs_kernel(float *g2n, uint64_t n, uint64_t th,
                                                           uint64_t seed, uint64_t tree,
                                                           double *block_max) {
    double mg = 0.0, mh = 0.0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        float2 v = reinterpret_cast<float2 *>(g2n)[i];
        if (!row_selected(i, th, seed, tree)) {
            v = make_float2(0.0f, 0.0f);
            reinterpret_cast<float2 *>(g2n)[i] = v;
        }
        mg = fmax(mg, finite_abs(v.x));
        mh = fmax(mh, finite_abs(v.y));
    }
    block_max2(mg, mh, block_max);
}

// The bounds of the whole array, and from them the quantizer scales.
__global__ void reduce_max_kernel(const double *block_max, uint32_t n, double *out,
                                  uint64_t n_rows, ScalesDev *scales) {
    __shared__ double sm[2][1024];
    double mg = 0.0, mh = 0.0;
    for (uint32_t i = threadIdx.x; i < n; i += 1024) {
        mg = fmax(mg, block_max[2 * i]);
        mh = fmax(mh, block_max[2 * i + 1]);
    }
    sm[0][threadIdx.x] = mg;
    sm[1][threadIdx.x] = mh;
    __syncthreads();
    for (uint32_t s = 512; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            sm[0][threadIdx.x] = fmax(sm[0][threadIdx.x], sm[0][threadIdx.x + s]);
            sm[1][threadIdx.x] = fmax(sm[1][threadIdx.x], sm[1][threadIdx.x + s]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        out[0] = sm[0][0];
        out[1] = sm[1][0];
        const ScalesDev prev = *scales;  // the scales a speculative pass used
        ScalesDev S{};
        S.max_abs[0] = sm[0][0];
        S.max_abs[1] = sm[1][0];
        S.status = (isfinite(S.max_abs[0]) && isfinite(S.max_abs[1]) && S.max_abs[0] >= 0.0 &&
                    S.max_abs[1] >= 0.0)
                       ? 0u
                       : 1u;
        for (int k = 0; k < 2; k++) {
            S.scale[k] = scale_from_bound(S.max_abs[k], n_rows);
            S.inv[k] = 1.0 / S.scale[k];
        }
        S.spec_miss = (prev.scale[0] == S.scale[0] && prev.scale[1] == S.scale[1]) ? 0u : 1u;
        *scales = S;
    }
}

// Scales the host chose (pairs it quantised itself).
__global__ void set_scales_kernel(ScalesDev *scales, double sg, double sh) {
    if (threadIdx.x != 0) return;
    ScalesDev S{};
    S.scale[0] = sg;
    S.scale[1] = sh;
    S.inv[0] = 1.0 / sg;
    S.inv[1] = 1.0 / sh;
    S.from_host = 1;
    *scales = S;
}

hipError_t launch_set_scales(ScalesDev *scales, double sg, double sh, hipStream_t s) {
    hipLaunchKernelGGL(set_scales_kernel, dim3(1), dim3(64), 0, s, scales, sg, sh);
    return hipGetLastError();
}

hipError_t launch_reduce_bounds(const double *block_max, uint32_t n_blocks, double *out_max,
                                uint64_t n_rows, ScalesDev *scales, hipStream_t s) {
    hipLaunchKernelGGL(reduce_max_kernel, dim3(1), dim3(1024), 0, s, block_max, n_blocks, out_max,
                       n_rows, scales);
    return hipGetLastError();
}

hipError_t launch_gpair_maxabs(float *g2n, uint64_t n, uint64_t th, uint64_t seed, uint64_t tree,
                               double *block_max, uint32_t n_blocks, hipStream_t s) {
    hipLaunchKernelGGL(gpair_maxabs_kernel, dim3(n_blocks), dim3(256), 0, s, g2n, n, th, seed,
                       tree, block_max);
    return hipGetLastError();
}

// `as i64` of Rust: saturating, NaN -> 0.
__device__ __forceinline__ int64_t sat_i64(double x) {
    if (isnan(x)) return 0;
    if (x >= 9223372036854775808.0) return (int64_t)0x7FFFFFFFFFFFFFFFll;
    if (x < -9223372036854775808.0) return (int64_t)0x8000000000000000ull;
    return (int64_t)x;
}

// GradQuantizer::to_fixed: round half away from zero of v * 2^k.
__global__ __launch_bounds__(256) void gpair_quantize_kernel(const float *g2n, uint64_t n,
                                                             const ScalesDev *scales, int64_t *out,
                                                             int64_t *block_sum) {
    const double sg = scales->scale[0], sh = scales->scale[1];
    uint64_t ag = 0, ah = 0;
    constexpr int U = 4;
    const uint64_t S = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t base = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; base < n;
         base += U * S) {
        float2 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint64_t i = base + u * S;
            v[u] = i < n ? reinterpret_cast<const float2 *>(g2n)[i] : make_float2(0.0f, 0.0f);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint64_t i = base + u * S;
            if (i >= n) continue;
            const int64_t qg = sat_i64(round((double)v[u].x * sg));
            const int64_t qh = sat_i64(round((double)v[u].y * sh));
            reinterpret_cast<longlong2 *>(out)[i] = make_longlong2(qg, qh);
            ag += (uint64_t)qg;
            ah += (uint64_t)qh;
        }
    }
    block_sum2(ag, ah, block_sum);
}

__global__ void reduce_sum_kernel(const int64_t *block_sum, uint32_t n, int64_t *out) {
    __shared__ int64_t sm[2][1024];
    uint64_t ag = 0, ah = 0;
    for (uint32_t i = threadIdx.x; i < n; i += 1024) {
        ag += (uint64_t)block_sum[2 * i];
        ah += (uint64_t)block_sum[2 * i + 1];
    }
    sm[0][threadIdx.x] = (int64_t)ag;
    sm[1][threadIdx.x] = (int64_t)ah;
    __syncthreads();
    for (uint32_t s = 512; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            sm[0][threadIdx.x] = wadd(sm[0][threadIdx.x], sm[0][threadIdx.x + s]);
            sm[1][threadIdx.x] = wadd(sm[1][threadIdx.x], sm[1][threadIdx.x + s]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        out[0] = sm[0][0];
        out[1] = sm[1][0];
    }
}

hipError_t launch_gpair_quantize(const float *g2n, uint64_t n, const ScalesDev *scales,
                                 int64_t *out, int64_t *block_sum, uint32_t n_blocks,
                                 int64_t *out_sum, hipStream_t s) {
    hipLaunchKernelGGL(gpair_quantize_kernel, dim3(n_blocks), dim3(256), 0, s, g2n, n, scales, out,
                       block_sum);
    if (out_sum)
        hipLaunchKernelGGL(reduce_sum_kernel, dim3(1), dim3(1024), 0, s, block_sum, n_blocks,
                           out_sum);
    return hipGetLastError();
}

// One column-major feature column [n_rows] of `width`-byte cells into its
// position (byte_off) of every row record of a tile.
__global__ void pack_feature_kernel(const uint8_t *col, uint64_t n_rows, uint32_t width,
                                    uint8_t *tile, uint32_t stride, uint32_t byte_off) {
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n_rows;
         r += (uint64_t)gridDim.x * blockDim.x) {
        uint8_t *dst = tile + r * stride + byte_off;
        if (width == 1) dst[0] = col[r];
        else *reinterpret_cast<uint16_t *>(dst) = reinterpret_cast<const uint16_t *>(col)[r];
    }
}

// One workgroup a column: counts in LDS over the sampled rows, then the
// largest count twice (lower code first on ties).
__global__ __launch_bounds__(256) void cat_hot_kernel(const CatColDev *cols, uint64_t n_rows,
                                                      uint32_t sample, uint32_t *out) {
    __shared__ uint32_t cnt[HOT_MAX_BINS];
    __shared__ uint32_t best_c[256], best_b[256];
    const CatColDev F = cols[blockIdx.x];
    const uint32_t nb = min(F.n_bins, HOT_MAX_BINS);
    for (uint32_t i = threadIdx.x; i < nb; i += 256) cnt[i] = 0;
    __syncthreads();
    const uint64_t m = min<uint64_t>(n_rows, sample);
    for (uint64_t i = threadIdx.x; i < m; i += 256) {
        const uint64_t r = m == n_rows ? i : i * n_rows / m;
        const uint32_t code = F.width == 1 ? (uint32_t)F.col[r]
                                           : (uint32_t) reinterpret_cast<const uint16_t *>(F.col)[r];
        if (code < nb) atomicAdd(&cnt[code], 1u);
    }
    __syncthreads();
    for (int pick = 0; pick < 2; pick++) {
        uint32_t bc = 0, bb = HOT_NONE;
        for (uint32_t i = threadIdx.x; i < nb; i += 256)
            if (cnt[i] > bc) {
                bc = cnt[i];
                bb = i;
            }
        best_c[threadIdx.x] = bc;
        best_b[threadIdx.x] = bb;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t c = 0, b = HOT_NONE;
            for (int t = 0; t < 256; t++)
                if (best_c[t] > c || (best_c[t] == c && c > 0 && best_b[t] < b)) {
                    c = best_c[t];
                    b = best_b[t];
                }
            out[4 * blockIdx.x + pick] = b;
            out[4 * blockIdx.x + 2 + pick] = c;
            if (b != HOT_NONE) cnt[b] = 0;
        }
        __syncthreads();
    }
}

hipError_t launch_cat_hot(const CatColDev *cols, uint32_t n_cols, uint64_t n_rows, uint32_t sample,
                          uint32_t *out, hipStream_t s) {
    if (n_cols == 0) return hipSuccess;
    hipLaunchKernelGGL(cat_hot_kernel, dim3(n_cols), dim3(256), 0, s, cols, n_rows, sample, out);
    return hipGetLastError();
}

hipError_t launch_pack_feature(const uint8_t *col, uint64_t n_rows, uint32_t width, uint8_t *tile,
                               uint32_t stride, uint32_t byte_off, hipStream_t s) {
    uint32_t blocks = (uint32_t)std::min<uint64_t>((n_rows + 255) / 256, 8192);
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(pack_feature_kernel, dim3(blocks), dim3(256), 0, s, col, n_rows, width,
                       tile, stride, byte_off);
    return hipGetLastError();
}

// Device binning (find_bin / quantize_value, src/data/columns.rs:335-356;
// categorical::code_to_bin): a workgroup bins a block of 64 rows x 64
// features. The block is read row by row (consecutive lanes, consecutive
// features of a row) into LDS, then binned column by column (consecutive
// lanes, consecutive rows of a feature), so both the matrix reads and the
// column writes are coalesced. A numeric value's bin is the number of cuts
// <= it (std::upper_bound), NaN the missing code, a categorical code v its
// own bin when 0 <= v < n_bins and else the unseen-category code.
constexpr uint32_t BIN_ROWS = 64, BIN_FEATS = 64;

__global__ __launch_bounds__(256) void bin_rows_kernel(const float *__restrict__ x,
                                                       uint64_t n_rows, uint32_t nf, uint64_t row0,
                                                       const BinFeatDev *__restrict__ feats) {
    __shared__ float blk[BIN_ROWS][BIN_FEATS + 1];
    const uint64_t rb = (uint64_t)blockIdx.x * BIN_ROWS;
    const uint32_t fb = blockIdx.y * BIN_FEATS;
    const uint32_t nr = (uint32_t)min<uint64_t>(BIN_ROWS, n_rows - rb);
    const uint32_t nfb = min(BIN_FEATS, nf - fb);
    for (uint32_t i = threadIdx.x; i < BIN_ROWS * BIN_FEATS; i += 256) {
        const uint32_t r = i / BIN_FEATS, f = i % BIN_FEATS;
        if (r < nr && f < nfb) blk[r][f] = x[(rb + r) * nf + fb + f];
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < BIN_ROWS * BIN_FEATS; i += 256) {
        const uint32_t f = i / BIN_ROWS, r = i % BIN_ROWS;
        if (r >= nr || f >= nfb) continue;
        const BinFeatDev F = feats[fb + f];
        const float v = blk[r][f];
        const uint32_t missing = F.width == 1 ? 0xFFu : 0xFFFFu;
        uint32_t bin;
        if (v != v) {
            bin = missing;
        } else if (F.categorical) {
            bin = (v >= 0.0f && v < (float)F.n_bins) ? (uint32_t)v : missing - 1u;
        } else {
            uint32_t lo = 0, hi = F.n_cuts;  // first cut > v
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (F.cuts[mid] <= v) lo = mid + 1;
                else hi = mid;
            }
            bin = lo;
        }
        const uint64_t row = row0 + rb + r;
        if (F.width == 1) F.col[row] = (uint8_t)bin;
        else reinterpret_cast<uint16_t *>(F.col)[row] = (uint16_t)bin;
    }
}

hipError_t launch_bin_rows(const float *x, uint64_t n_rows, uint32_t n_features, uint64_t row0,
                           const BinFeatDev *feats, hipStream_t s) {
    if (n_rows == 0 || n_features == 0) return hipSuccess;
    const dim3 grid((uint32_t)((n_rows + BIN_ROWS - 1) / BIN_ROWS),
                    (n_features + BIN_FEATS - 1) / BIN_FEATS);
    hipLaunchKernelGGL(bin_rows_kernel, grid, dim3(256), 0, s, x, n_rows, n_features, row0, feats);
    return hipGetLastError();
}

// Packed tiles: a workgroup packs 256 consecutive rows of one row bundle
// (blockIdx.y; the 128 / (16 W) consecutive tiles sharing it, every tile's
// stride the bundle's pitch). Phase 1 reads each of the bundle's columns for
// the 256 rows (consecutive lanes, consecutive cells) into the rows'
// records in LDS; phase 2 writes the 256 records, consecutive lanes writing
// consecutive 16-byte pieces of the bundle's contiguous rows. Empty cells
// are zero.
constexpr uint32_t PACK_ROWS = 256;
constexpr uint32_t PACK_LDS_STRIDE = 33;  // dwords a row in LDS (32 + 1: no bank conflicts)

template <int W>
__global__ __launch_bounds__(256) void pack_tiles_kernel(const PackTileDev *__restrict__ tiles,
                                                         uint32_t n_tiles, uint64_t n_rows) {
    constexpr uint32_t PER = 8 / W;       // tiles a bundle (16 cells each: 128 bytes a row)
    constexpr uint32_t CPD = 4 / W;       // cells a dword
    __shared__ uint32_t rec[PACK_ROWS * PACK_LDS_STRIDE];
    const uint32_t t0 = blockIdx.y * PER;
    const uint32_t nt = min(PER, n_tiles - t0);
    const uint64_t r0 = (uint64_t)blockIdx.x * PACK_ROWS;
    const uint32_t tid = threadIdx.x;
    const bool in = r0 + tid < n_rows;
    const uint64_t r = in ? r0 + tid : r0;  // a valid row for every lane's loads
    // Phase 1: thread tid builds row r0 + tid's record, 64 cells at a time:
    // every cell loads first (an empty cell, or a tile past the last, from a
    // valid column), so the loads issue back to back; then the dwords are
    // assembled, empty cells and rows past the end masked to zero.
    constexpr uint32_t GT = 64 / 16;  // tiles loaded together
#pragma unroll
    for (uint32_t g = 0; g < PER; g += GT) {
        uint32_t v[GT][16];
#pragma unroll
        for (uint32_t j = 0; j < GT; j++) {
            const PackTileDev &T = tiles[t0 + (g + j < nt ? g + j : 0u)];
#pragma unroll
            for (int k = 0; k < 16; k++)
                v[j][k] = W == 1 ? (uint32_t)T.col[k][r]
                                 : (uint32_t)reinterpret_cast<const uint16_t *>(T.col[k])[r];
        }
#pragma unroll
        for (uint32_t j = 0; j < GT; j++) {
            const uint32_t live = g + j < nt && in ? tiles[t0 + g + j].live : 0u;
#pragma unroll
            for (uint32_t q = 0; q < 16 / CPD; q++) {
                uint32_t d = 0;
#pragma unroll
                for (uint32_t c = 0; c < CPD; c++) {
                    const uint32_t k = q * CPD + c;
                    if (live >> k & 1u) d |= v[j][k] << (c * 8 * W);
                }
                rec[tid * PACK_LDS_STRIDE + (g + j) * (16 / CPD) + q] = d;
            }
        }
    }
    __syncthreads();
    // Phase 2: the bundle's rows r0.. are contiguous at pitch bytes each.
    const uint32_t pitch = tiles[t0].stride;  // 16 W nt rounded up to a power of two
    const uint32_t quads = pitch / 16;        // 16-byte pieces a row
    const uint64_t rows = min<uint64_t>(PACK_ROWS, n_rows - r0);
    uint8_t *base = tiles[t0].out + r0 * pitch;
    for (uint32_t i = tid; i < rows * quads; i += 256) {
        const uint32_t row = i / quads, qd = i % quads;
        const uint32_t *src = rec + row * PACK_LDS_STRIDE + 4 * qd;
        reinterpret_cast<uint4 *>(base)[i] = make_uint4(src[0], src[1], src[2], src[3]);
    }
}

hipError_t launch_pack_tiles(const PackTileDev *tiles, uint32_t n_tiles, uint32_t width,
                             uint64_t n_rows, hipStream_t s) {
    if (n_tiles == 0 || n_rows == 0) return hipSuccess;
    if (width != 1 && width != 2) return hipErrorInvalidValue;
    const uint32_t per = 8 / width;
    const dim3 grid((uint32_t)((n_rows + PACK_ROWS - 1) / PACK_ROWS), (n_tiles + per - 1) / per);
    if (width == 1)
        hipLaunchKernelGGL(pack_tiles_kernel<1>, grid, dim3(256), 0, s, tiles, n_tiles, n_rows);
    else
        hipLaunchKernelGGL(pack_tiles_kernel<2>, grid, dim3(256), 0, s, tiles, n_tiles, n_rows);
    return hipGetLastError();
}

// ======================================================================
// device-grown depthwise trees
// ======================================================================
// The host enqueues every level of a depthwise tree without waiting: each
// level's decision kernel reads the split packets where the split scan left
// them and plans the partition and the children exactly as the host grower
// would (build_tree, src/training/mod.rs:3357-4565).

// The root of a device-grown tree. Block 0 takes the root sum (staged from
// the host, or the wrapping sum of the quantisation's per-block sums) and
// initialises the state, the root's level node, split node and tree node;
// every block clears its share of `clear` (the root's histogram slot when it
// accumulates atomically).
__global__ __launch_bounds__(1024) void grow_prep_kernel(
    GrowParamsDev G, const int64_t *root, const int64_t *block_sums, uint32_t n_blocks,
    uint32_t root_slot, LNodeDev *level, SplitNodeDev *root_split, TreeNodeDev *tree,
    GrowState *st, int64_t *clear, uint64_t clear_words) {
    __shared__ int64_t wsum[2][16];
    if (clear)
        for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < clear_words;
             i += (uint64_t)gridDim.x * blockDim.x)
            clear[i] = 0;
    if (blockIdx.x != 0) return;
    int64_t rg, rh;
    if (block_sums) {
        uint64_t ag = 0, ah = 0;
        for (uint32_t i = threadIdx.x; i < n_blocks; i += blockDim.x) {
            ag += (uint64_t)block_sums[2 * i];
            ah += (uint64_t)block_sums[2 * i + 1];
        }
        for (int off = 32; off > 0; off >>= 1) {
            ag += (uint64_t)__shfl_xor((long long)ag, off, 64);
            ah += (uint64_t)__shfl_xor((long long)ah, off, 64);
        }
        if ((threadIdx.x & 63) == 0) {
            wsum[0][threadIdx.x >> 6] = (int64_t)ag;
            wsum[1][threadIdx.x >> 6] = (int64_t)ah;
        }
        __syncthreads();
        if (threadIdx.x != 0) return;
        ag = ah = 0;
        for (uint32_t w = 0; w < blockDim.x / 64; w++) {
            ag += (uint64_t)wsum[0][w];
            ah += (uint64_t)wsum[1][w];
        }
        rg = (int64_t)ag;
        rh = (int64_t)ah;
    } else {
        if (threadIdx.x != 0) return;
        rg = root[0];
        rh = root[1];
    }
    load_scales(G.sp);
    GrowState s{};
    s.n_level = 1;
    s.tree_size = 1;
    s.leaf_count = 1;
    s.scales = *G.sp.scales;
    s.error = s.scales.status ? 2u : 0u;
    *st = s;
    LNodeDev r{};
    r.tree_id = 0;
    r.row_off = 0;
    r.row_len = G.n_rows;
    r.slot = root_slot;
    r.sum_g = rg;
    r.sum_h = rh;
    r.lower = -3.40282347e38f;
    r.upper = 3.40282347e38f;
    level[0] = r;
    SplitNodeDev sn{};
    sn.sum_g = rg;
    sn.sum_h = rh;
    sn.lower = r.lower;
    sn.upper = r.upper;
    sn.slot = root_slot;
    root_split[0] = sn;
    const double g = (double)rg * G.sp.inv_g, h = (double)rh * G.sp.inv_h;
    TreeNodeDev t{};
    t.left = t.right = -1;
    t.flags = 1;
    t.leaf_value = xgb_weight(g, h, G.sp) * G.learning_rate;
    t.sum_hess = (float)h;
    t.pad[1] = NO_SLOT;  // no leaf position yet
    tree[0] = t;
}

hipError_t launch_grow_prep(const GrowParamsDev &G, const int64_t *root, const int64_t *block_sums,
                            uint32_t n_blocks, uint32_t root_slot, LNodeDev *level,
                            SplitNodeDev *root_split, TreeNodeDev *tree, GrowState *st,
                            int64_t *clear, uint64_t clear_words, hipStream_t s) {
    const uint32_t blocks =
        clear ? (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>((clear_words + 1023) / 1024, 256))
              : 1u;
    hipLaunchKernelGGL(grow_prep_kernel, dim3(blocks), dim3(1024), 0, s, G, root, block_sums,
                       n_blocks, root_slot, level, root_split, tree, st, clear, clear_words);
    return hipGetLastError();
}

// One level of a device-grown tree (one workgroup, each thread a run of the
// level's nodes in order):
//  - the max_leaves budget: the first `remaining` nodes with a split split;
//  - a node that does not split is a leaf (leaf table, when it has rows);
//  - a split node s (s-th in order) gets children tree_size + 2s, + 1 with
//    the weights, monotone bounds and Hessians of Tree::split_leaf and
//    child_leaves (src/training/mod.rs:5069-5094), its partition request,
//    and, when the children are evaluated, the lowest free histogram slot
//    for the smaller child (the larger one takes over the node's slot).
__global__ __launch_bounds__(1024) void grow_decide_kernel(
    GrowParamsDev G, uint32_t depth, SplitPacketDev *pk, uint64_t *pk_cats,
    const LNodeDev *level, TreeNodeDev *tree, uint64_t *tree_cats, const int8_t *monotone,
    const DevColumn *cols, PartReqDev *reqs, PairDev *pairs, uint32_t *triples, LeafDev *leaves,
    float *leaf_vals, GrowState *st, FusedArgmaxDev A) {
    __shared__ uint32_t buf[1024];
    __shared__ uint32_t held[MAX_GROW_SLOTS / 32];
    __shared__ uint16_t freelist[MAX_GROW_SLOTS];
    load_scales(G.sp);
    const uint32_t tid = threadIdx.x;
    // The fields this launch reads, one by one: a copy of the whole state
    // would live in scratch memory.
    struct {
        uint32_t n_level, leaf_count, tree_size, tree_cat_words, n_leaves, error;
    } S0;
    S0.n_level = st->n_level;
    S0.leaf_count = st->leaf_count;
    S0.tree_size = st->tree_size;
    S0.tree_cat_words = st->tree_cat_words;
    S0.n_leaves = st->n_leaves;
    S0.error = st->error;
    __syncthreads();  // every thread has read the state before thread 0 rewrites it
    const uint32_t n = S0.n_level;
    const uint32_t per = (n + 1023) / 1024;
    const uint32_t i0 = min(tid * per, n), i1 = min(i0 + per, n);
    // With at most 1024 nodes each thread's packet and node stay in
    // registers for every pass.
    // A.cands set: the packets are made here from the split scan's
    // candidates (split_node_kernel's work), else read.
    // With few enough candidates, the workgroup first stages every
    // (node, feature) candidate's gain in LDS (-1 when none: found
    // candidates' gains are above MIN_GAIN_EPS), all loads in flight at
    // once; each node's argmax then reads LDS.
    __shared__ float cand_gain[DECIDE_CAND_LDS];
    const uint32_t nfe = G.sp.n_feats;
    const bool staged = A.cands && per == 1 && (uint64_t)n * nfe <= DECIDE_CAND_LDS;
    if (staged) {
#pragma unroll
        for (uint32_t k = 0; k < DECIDE_CAND_LDS / 1024; k++) {
            const uint32_t q = tid + k * 1024;
            if (q < n * nfe) {
                const float g = A.cands[q].gain;
                const uint32_t f = A.cands[q].found;
                cand_gain[q] = f ? g : -1.0f;
            }
        }
        __syncthreads();
    }
    // Each node's first feature of the largest gain (as split_packet_serial
    // picks it) from the staged gains: with many features by a group of gl
    // lanes of one wave (the workgroup's threads shared among the nodes),
    // reduced by shuffles, ord_sh[i] holding node i's feature + 1 (0: none);
    // with few, by the node's own thread (the group's barrier and shuffles
    // cost more than it saves: 10.5M x 28 lost 0.3 %, 2M x 100 gained 0.5 %).
    __shared__ uint32_t ord_sh[1024];
    const bool grouped = staged && nfe > 64;
    if (grouped) {
        uint32_t gl = 64;
        while (gl > 1 && gl * n > 1024) gl >>= 1;
        const uint32_t i = tid / gl, sub = tid % gl;
        float best = 0.0f;
        uint32_t ord = 0xFFFFFFFFu;
        if (i < n)
            for (uint32_t j = sub; j < nfe; j += gl) {
                const float g = cand_gain[i * nfe + j];
                if (g > best) {  // j ascends: ties keep the lower feature
                    best = g;
                    ord = j;
                }
            }
        for (uint32_t off = gl >> 1; off > 0; off >>= 1) {
            const float ob = __shfl_xor(best, (int)off, 64);
            const uint32_t oo = __shfl_xor(ord, (int)off, 64);
            if (ob > best || (ob == best && oo < ord)) {
                best = ob;
                ord = oo;
            }
        }
        if (i < n && sub == 0) ord_sh[i] = best > 0.0f ? ord + 1 : 0u;
        __syncthreads();
    }
    auto make_pk = [&](uint32_t i) -> SplitPacketDev {
        if (staged) {
            uint32_t found = 0, ord = 0;
            if (grouped) {
                const uint32_t o = ord_sh[i];
                found = o ? 1u : 0u;
                ord = o ? o - 1 : 0u;
            } else {
                float best = 0.0f;
                for (uint32_t j = 0; j < nfe; j++) {
                    const float g = cand_gain[i * nfe + j];
                    if (g > best) {
                        best = g;
                        ord = j;
                        found = 1;
                    }
                }
            }
            return split_packet(A.cands + (size_t)i * nfe, A.feats, G.sp, i, found, ord, A.nodes,
                                A.cat_scratch, pk_cats, G.cw);
        }
        return A.cands ? split_packet_serial(A.cands, A.feats, G.sp, i, A.nodes, A.cat_scratch,
                                             pk_cats, G.cw)
                       : pk[i];
    };
    SplitPacketDev myP{};
    LNodeDev myL{};
    TreeNodeDev myT{};
    int myMono = 0;
    DevColumn myCol{};
    if (per == 1 && i0 < n) myL = level[i0];
    // The packets, one inlined builder (the kernel's code is fetched once a
    // level: its size is latency): held in registers with one node a
    // thread, else stored to pk for the passes below.
    if (A.cands || per == 1)
        for (uint32_t i = i0; i < i1; i++) {
            const SplitPacketDev P = make_pk(i);
            if (per == 1) myP = P;
            else pk[i] = P;
        }
    if (per == 1 && i0 < n) {
        // What the node's pass below reads, requested while the scans run.
        myT = tree[myL.tree_id];
        if (myP.found) {
            myMono = monotone[myP.feat];
            myCol = cols[myP.feat];
        }
    }
    auto pk_at = [&](uint32_t i) -> SplitPacketDev { return per == 1 ? myP : pk[i]; };
    auto lv_at = [&](uint32_t i) -> LNodeDev { return per == 1 ? myL : level[i]; };

    uint32_t f_before, tot_found, l_before, tot_leaves, c_before, tot_chunks, n_split;
    __shared__ uint32_t buf3[3][32];
    if (!G.max_leaves) {
        // No leaf cap: every node with a split splits, so the split nodes,
        // leaves and partition chunks take one scan.
        uint32_t v[3] = {0u, 0u, 0u}, t[3];
        for (uint32_t i = i0; i < i1; i++) {
            const uint32_t len = lv_at(i).row_len;
            if (pk_at(i).found) {
                v[0]++;
                v[2] += (len + PART_CHUNK - 1) / PART_CHUNK;
            } else if (len) {
                v[1]++;
            }
        }
        block_scan_n<3>(v, buf3, t);
        f_before = v[0];
        tot_found = t[0];
        l_before = v[1];
        tot_leaves = t[1];
        c_before = v[2];
        tot_chunks = t[2];
        n_split = tot_found;
    } else {
        uint32_t nf = 0;
        for (uint32_t i = i0; i < i1; i++) nf += pk_at(i).found ? 1u : 0u;
        f_before = block_scan_1024(nf, buf, tot_found);
        const uint32_t remaining =
            G.max_leaves > S0.leaf_count ? G.max_leaves - S0.leaf_count : 0u;
        n_split = min(tot_found, remaining);
        uint32_t v[2] = {0u, 0u}, t[2];
        uint32_t fr = f_before;
        for (uint32_t i = i0; i < i1; i++) {
            const bool found = pk_at(i).found != 0;
            const uint32_t len = lv_at(i).row_len;
            if (found && fr < n_split) v[1] += (len + PART_CHUNK - 1) / PART_CHUNK;
            else if (len) v[0]++;
            if (found) fr++;
        }
        block_scan_n<2>(v, buf3, t);
        l_before = v[0];
        tot_leaves = t[0];
        c_before = v[1];
        tot_chunks = t[1];
    }
    const uint32_t leaf_count = S0.leaf_count + n_split;
    bool evaluated =
        n_split > 0 && depth + 1 < G.max_depth && !(G.max_leaves && leaf_count >= G.max_leaves);

    bool slots_short = false;
    if (evaluated) {
        const uint32_t words = (G.n_slots + 31) / 32;
        for (uint32_t w = tid; w < words; w += 1024) held[w] = 0;
        __syncthreads();
        uint32_t fr = f_before;
        for (uint32_t i = i0; i < i1; i++) {
            if (!pk_at(i).found) continue;
            const uint32_t slot = lv_at(i).slot;
            if (fr < n_split) atomicOr(&held[slot >> 5], 1u << (slot & 31));
            fr++;
        }
        __syncthreads();
        const uint32_t sp = (G.n_slots + 1023) / 1024;
        const uint32_t s0 = min(tid * sp, G.n_slots), s1 = min(s0 + sp, G.n_slots);
        uint32_t nfree = 0;
        for (uint32_t q = s0; q < s1; q++) nfree += ((held[q >> 5] >> (q & 31)) & 1u) ? 0u : 1u;
        uint32_t tot_free;
        uint32_t fb = block_scan_1024(nfree, buf, tot_free);
        for (uint32_t q = s0; q < s1; q++)
            if (!((held[q >> 5] >> (q & 31)) & 1u)) freelist[fb++] = (uint16_t)q;
        __syncthreads();
        if (tot_free < n_split) {
            slots_short = true;
            evaluated = false;
        }
    }

    uint32_t fr = f_before, lr = l_before, cb = c_before;
    for (uint32_t i = i0; i < i1; i++) {
        const SplitPacketDev P = pk_at(i);
        const LNodeDev L = lv_at(i);
        const bool split = P.found && fr < n_split;
        if (split) {
            const uint32_t s = fr;
            const uint32_t lid = S0.tree_size + 2 * s, rid = lid + 1;
            const double gl = (double)P.left[0] * G.sp.inv_g, hl = (double)P.left[1] * G.sp.inv_h;
            const double gr = (double)P.right[0] * G.sp.inv_g,
                         hr = (double)P.right[1] * G.sp.inv_h;
            const float wl = apply_bounds(xgb_weight(gl, hl, G.sp), L.lower, L.upper);
            const float wr = apply_bounds(xgb_weight(gr, hr, G.sp), L.lower, L.upper);
            const int mono = per == 1 ? myMono : monotone[P.feat];
            const float mid = (wl + wr) / 2.0f;
            float llo = L.lower, lhi = L.upper, rlo = L.lower, rhi = L.upper;
            if (mono < 0) {
                llo = mid;
                rhi = mid;
            } else if (mono > 0) {
                lhi = mid;
                rlo = mid;
            }
            TreeNodeDev t = per == 1 ? myT : tree[L.tree_id];
            t.feat = P.feat;
            t.bin = P.bin;
            t.left = (int32_t)lid;
            t.right = (int32_t)rid;
            t.pad[0] = __float_as_uint(t.leaf_value);  // its value had it stayed a leaf
            t.leaf_value = 0.0f;
            t.gain = P.gain;
            t.flags = (P.missing_left ? 2u : 0u) | (P.is_cat ? 4u : 0u);
            t.cat_off = S0.tree_cat_words + s * G.cw;
            t.n_cat_words = P.is_cat ? P.n_cat_words : 0u;
            for (uint32_t w = 0; w < t.n_cat_words; w++)
                tree_cats[t.cat_off + w] = pk_cats[P.cat_offset + w];
            tree[L.tree_id] = t;
            TreeNodeDev a{}, b{};
            a.left = a.right = b.left = b.right = -1;
            a.flags = b.flags = 1;
            a.pad[1] = b.pad[1] = NO_SLOT;  // no leaf position yet
            a.leaf_value = wl * G.learning_rate;
            a.sum_hess = (float)hl;
            b.leaf_value = wr * G.learning_rate;
            b.sum_hess = (float)hr;
            tree[lid] = a;
            tree[rid] = b;
            const DevColumn col = per == 1 ? myCol : cols[P.feat];
            PartReqDev q{};
            q.row_off = L.row_off;
            q.row_len = L.row_len;
            q.chunk_begin = cb;
            q.count_base = cb;
            q.n_chunks = (L.row_len + PART_CHUNK - 1) / PART_CHUNK;
            q.data = col.data;
            q.stride = col.width;
            q.byte_off = 0;
            q.width = col.width;
            q.missing = col.missing;
            q.bin = P.bin;
            q.missing_left = P.missing_left;
            q.cat_off = P.cat_offset;
            q.n_cat_words = P.is_cat ? P.n_cat_words : 0u;
            reqs[s] = q;
            if (G.part_cur) G.part_cur[(uint64_t)s * PART_CURSOR_STRIDE] = 0ull;
            cb += q.n_chunks;
            PairDev d{};
            d.req = L.row_len ? s : NO_SLOT;
            d.row_off = L.row_off;
            d.row_len = L.row_len;
            d.parent_slot = L.slot;
            d.new_slot = evaluated ? (uint32_t)freelist[s] : NO_SLOT;
            d.eval_index = evaluated ? s : NO_SLOT;
            d.lower[0] = llo;
            d.lower[1] = rlo;
            d.upper[0] = lhi;
            d.upper[1] = rhi;
            d.left_sum[0] = P.left[0];
            d.left_sum[1] = P.left[1];
            d.right_sum[0] = P.right[0];
            d.right_sum[1] = P.right[1];
            d.left_id = lid;
            d.right_id = rid;
            pairs[s] = d;
            if (evaluated) {
                triples[3 * s] = L.slot;
                triples[3 * s + 1] = L.slot;
                triples[3 * s + 2] = freelist[s];
            }
        } else if (L.row_len) {
            const uint32_t k = S0.n_leaves + lr++;
            LeafDev lf{};
            lf.row_off = L.row_off;
            lf.row_len = L.row_len;
            lf.value = per == 1 ? myT.leaf_value : tree[L.tree_id].leaf_value;
            lf.id = k;
            lf.arena = depth & 1u;
            leaves[k] = lf;
            leaf_vals[k] = lf.value;
            tree[L.tree_id].pad[1] = k;  // the leaf's position
        }
        if (P.found) fr++;
    }
    __syncthreads();
    if (tid == 0) {
        st->n_split = n_split;
        st->part_chunks = tot_chunks;
        st->n_eval = evaluated ? n_split : 0u;
        st->tree_size = S0.tree_size + 2 * n_split;
        st->leaf_count = leaf_count;
        st->n_leaves = S0.n_leaves + tot_leaves;
        st->tree_cat_words = S0.tree_cat_words + n_split * G.cw;
        st->error = S0.error | (slots_short ? 1u : 0u);
    }
}

hipError_t launch_grow_decide(const GrowParamsDev &G, uint32_t depth, SplitPacketDev *pk,
                              uint64_t *pk_cats, const LNodeDev *level, TreeNodeDev *tree,
                              uint64_t *tree_cats, const int8_t *monotone, const DevColumn *cols,
                              PartReqDev *reqs, PairDev *pairs, uint32_t *triples,
                              LeafDev *leaves, float *leaf_vals, GrowState *st,
                              const FusedArgmaxDev &A, hipStream_t s) {
    if (G.n_slots > MAX_GROW_SLOTS) return hipErrorInvalidValue;
    hipLaunchKernelGGL(grow_decide_kernel, dim3(1), dim3(1024), 0, s, G, depth, pk, pk_cats, level,
                       tree, tree_cats, monotone, cols, reqs, pairs, triples, leaves, leaf_vals,
                       st, A);
    return hipGetLastError();
}

// Chunk layout of the finished leaf table and the rows it covers.
__global__ __launch_bounds__(1024) void leaf_plan_kernel(LeafDev *leaves, GrowState *st) {
    __shared__ uint32_t buf[1024];
    __shared__ unsigned long long cov_sh;
    const uint32_t n = st->n_leaves;
    if (threadIdx.x == 0) cov_sh = 0;
    const uint32_t per = (n + 1023) / 1024;
    const uint32_t i0 = min(threadIdx.x * per, n), i1 = min(i0 + per, n);
    uint32_t nc = 0;
    unsigned long long cov = 0;
    for (uint32_t i = i0; i < i1; i++) {
        nc += (leaves[i].row_len + PART_CHUNK - 1) / PART_CHUNK;
        cov += leaves[i].row_len;
    }
    uint32_t total;
    uint32_t cb = block_scan_1024(nc, buf, total);
    for (uint32_t i = i0; i < i1; i++) {
        leaves[i].chunk_begin = cb;
        cb += (leaves[i].row_len + PART_CHUNK - 1) / PART_CHUNK;
    }
    atomicAdd(&cov_sh, cov);
    __syncthreads();
    if (threadIdx.x == 0) {
        st->leaf_chunks = total;
        st->covered = cov_sh;
    }
}

// Leaves of a device-grown tree by walking it in row order, when every tree
// feature sits in one row bundle: the row's record gives each split's cell
// (the partition's go-left rule: missing -> default direction, categorical
// -> not in the right-going set, else bin < split bin). ids[row] is the
// leaf's position among the leaves in node-id order; the margin gets the
// leaf value with the same f32 addition as apply_leaves (or delta[row] =
// value without an objective). This replaces the last level's partition and
// the scattered leaf-id writes. Workgroup 0 also writes the leaf values by
// position and the leaf count.
template <int IDB, int PB>
__global__ __launch_bounds__(256) void tree_leaves_kernel(
    const uint8_t *bundle, uint64_t n_rows, TreeNodeDev *tree, const uint64_t *tree_cats,
    const uint16_t *feat_off, GrowState *st, void *ids, float *margin, float *delta,
    float *leaf_vals) {
    __shared__ uint32_t buf[32];
    // Node: meta (bits 0-5 cell offset, 6: 16-bit cell, 7: leaf, 8: missing
    // goes left, 9: categorical, 10: an 8-bit cell without a missing code),
    // split bin, left, right.
    __shared__ ushort4 s_node[MAX_WALK_NODES];
    __shared__ uint16_t s_leaf[MAX_WALK_NODES];
    __shared__ uint32_t s_cat[MAX_WALK_NODES];
    __shared__ uint8_t s_ncw[MAX_WALK_NODES];
    __shared__ float s_val[MAX_WALK_NODES];
    const uint32_t n = st->tree_size;
    __syncthreads();  // every thread has read the size before workgroup 0 updates the state
    uint32_t carry = 0;
    for (uint32_t base = 0; base < n; base += blockDim.x) {
        const uint32_t k = base + threadIdx.x;
        uint32_t lf = 0;
        if (k < n) {
            // The fields the walk uses, one by one: workgroup 0 writes each
            // leaf's position (pad[1]) below, which no workgroup reads.
            const TreeNodeDev &t = tree[k];
            const uint32_t flags = t.flags;
            lf = flags & 1u;
            const uint32_t fo = lf ? 0u : feat_off[t.feat];
            const uint32_t meta = (fo & 0x3Fu) | ((fo & 0x8000u) ? 0x40u : 0u) | (lf << 7) |
                                  ((flags & 2u) << 7) | ((flags & 4u) << 7) |
                                  ((fo & 0x4000u) ? 0x400u : 0u);
            s_node[k] = make_ushort4((uint16_t)meta, (uint16_t)t.bin, (uint16_t)t.left,
                                     (uint16_t)t.right);
            s_cat[k] = t.cat_off;
            s_ncw[k] = (uint8_t)t.n_cat_words;
            s_val[k] = t.leaf_value;
        }
        uint32_t tot;
        const uint32_t before = carry + block_scan(lf, buf, tot);
        if (k < n && lf) {
            s_leaf[k] = (uint16_t)before;
            if (blockIdx.x == 0) {
                leaf_vals[before] = s_val[k];
                tree[k].pad[1] = before;  // the leaf's position
            }
        }
        carry += tot;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        st->n_leaves = carry;
        st->covered = n_rows;
    }
    __syncthreads();
    for (uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n_rows;
         r += (uint64_t)gridDim.x * blockDim.x) {
        // The row's whole record in registers, then cells by select.
        uint32_t rec[PB];
#pragma unroll
        for (int q = 0; q < PB / 4; q++) {
            const uint4 v = reinterpret_cast<const uint4 *>(bundle + r * (PB * 4))[q];
            rec[4 * q] = v.x;
            rec[4 * q + 1] = v.y;
            rec[4 * q + 2] = v.z;
            rec[4 * q + 3] = v.w;
        }
        // The margin's load is issued before the walk, its use after (no
        // margin: leaf ids only, the values are added later).
        const float m = IDB && margin ? margin[r] : 0.0f;
        uint32_t node = 0;
        ushort4 nd = s_node[0];
        while (!(nd.x & 0x80u)) {
            const uint32_t off = nd.x & 0x3Fu;
            const uint32_t qi = off >> 2;
            uint32_t word = rec[0];
#pragma unroll
            for (int q = 1; q < PB; q++) word = (qi == (uint32_t)q) ? rec[q] : word;
            const bool w2 = (nd.x & 0x40u) != 0;
            const uint32_t bin = (word >> ((off & 3u) * 8u)) & (w2 ? 0xFFFFu : 0xFFu);
            // an 8-bit column of 256 bins has no missing code (bit 10)
            const uint32_t missing = w2 ? 0xFFFFu : ((nd.x & 0x400u) ? 0x100u : 0xFFu);
            bool gl;
            if (bin == missing) {
                gl = (nd.x & 0x100u) != 0;
            } else if (nd.x & 0x200u) {
                const uint32_t w = bin >> 6;
                gl = !(w < s_ncw[node] && ((tree_cats[s_cat[node] + w] >> (bin & 63)) & 1ull));
            } else {
                gl = bin < nd.y;
            }
            node = gl ? nd.z : nd.w;
            nd = s_node[node];
        }
        if (IDB == 0) {
            delta[r] = s_val[node];
        } else {
            if (IDB == 1) static_cast<uint8_t *>(ids)[r] = (uint8_t)s_leaf[node];
            else static_cast<uint16_t *>(ids)[r] = s_leaf[node];
            if (margin) margin[r] = m + s_val[node];
        }
    }
}

template <int IDB>
static void launch_walk_pb(uint32_t pitch, dim3 g, hipStream_t s, const uint8_t *bundle,
                           uint64_t n_rows, TreeNodeDev *tree, const uint64_t *tree_cats,
                           const uint16_t *feat_off, GrowState *st, void *ids, float *margin,
                           float *delta, float *leaf_vals) {
    if (pitch == 16)
        hipLaunchKernelGGL((tree_leaves_kernel<IDB, 4>), g, dim3(256), 0, s, bundle, n_rows, tree,
                           tree_cats, feat_off, st, ids, margin, delta, leaf_vals);
    else if (pitch == 32)
        hipLaunchKernelGGL((tree_leaves_kernel<IDB, 8>), g, dim3(256), 0, s, bundle, n_rows, tree,
                           tree_cats, feat_off, st, ids, margin, delta, leaf_vals);
    else
        hipLaunchKernelGGL((tree_leaves_kernel<IDB, 16>), g, dim3(256), 0, s, bundle, n_rows,
                           tree, tree_cats, feat_off, st, ids, margin, delta, leaf_vals);
}

hipError_t launch_tree_leaves(const uint8_t *bundle, uint32_t pitch, uint64_t n_rows,
                              TreeNodeDev *tree, const uint64_t *tree_cats,
                              const uint16_t *feat_off, GrowState *st, void *ids, int id_bytes,
                              float *margin, float *delta, float *leaf_vals, hipStream_t s) {
    if (pitch != 16 && pitch != 32 && pitch != 64) return hipErrorInvalidValue;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((n_rows + 255) / 256, 2048);
    if (blocks == 0) return hipSuccess;
    const dim3 g(blocks);
    if (id_bytes == 1)
        launch_walk_pb<1>(pitch, g, s, bundle, n_rows, tree, tree_cats, feat_off, st, ids, margin,
                          delta, leaf_vals);
    else if (id_bytes == 2)
        launch_walk_pb<2>(pitch, g, s, bundle, n_rows, tree, tree_cats, feat_off, st, ids, margin,
                          delta, leaf_vals);
    else
        launch_walk_pb<0>(pitch, g, s, bundle, n_rows, tree, tree_cats, feat_off, st, ids, margin,
                          delta, leaf_vals);
    return hipGetLastError();
}

hipError_t launch_leaf_plan(LeafDev *leaves, GrowState *st, hipStream_t s) {
    hipLaunchKernelGGL(leaf_plan_kernel, dim3(1), dim3(1024), 0, s, leaves, st);
    return hipGetLastError();
}

}  // namespace fbh
