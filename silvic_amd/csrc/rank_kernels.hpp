// rank_kernels.hpp - LambdaRank-NDCG gradients on the device, bit for bit the host's f64 ones (lambdarank.hpp,
// which follows crates/silvic-core/src/objective/lambdarank.rs:190-420).
//
// One wave per query (k_rank_pairs): the query's rows are ranked by score (descending, ties by row) with a bitonic
// sort in LDS, then every row i above the truncation level takes its pairs (i, j), j > i, in order. A ballot over the
// ranks j marks the pairs the host takes (below the first -inf score, a different label); the marked lanes compute
// their pair terms (the arithmetic is srocm_rank's, shared with the host), and lane j adds its own term to rank j's
// sums, so each rank's "as j" sums are taken over i in increasing order, as the host takes them. Row i's own sums and
// the query's lambda sum are running f64 sums in pair order: the marked terms are listed in LDS in j order, and three
// lanes (lambda, hessian, lambda sum) each add up their list, so every sum has the host's operation sequence. The
// table reads of row i + 1 are issued before row i is added up, so their latency hides behind that serial sum.
//
// The unscaled sums go to per-row f64 buffers and the lambda sum to a per-query buffer. k_rank_factor makes each
// query's normalization factor log2(1 + s) / s from both doubles around log2(1 + s) (log2_dd.hpp: the C library's
// log2, which the host takes, is one of them), and k_rank_scale keeps it where both give every row of the query the
// same f32 gradient and hessian, so the scaled gradients equal the host's to the last bit; a query where they could
// differ raises a flag, and the host then makes the iteration's factors itself.
#pragma once

#include "lambdarank.hpp"
#include "log2_dd.hpp"

#include <hip/hip_runtime.h>

namespace srocm {

struct RankArgs {
    const float *scores, *label;
    const uint32_t *bounds;        // num_queries + 1 row offsets
    const double *inv_max_dcg;     // per query
    const double *label_gain;      // per label
    const double *table;           // the sigmoid table (srocm_rank::SIGMOID_BINS)
    const double *discount;        // 1 / log2(2 + rank), srocm_rank::DISCOUNT_TABLE of them
    double sigmoid, sigmoid2, min_input, max_input, idx_factor;
    uint32_t norm, truncation;
    double *lam, *hes;             // per row: the unscaled lambda and hessian sums
    double *qsum;                  // per query: the lambda sum
    const uint32_t *queries;       // the queries this launch takes, one a block (blockIdx.x's is queries[blockIdx.x])
    uint32_t *flag;                // when set, cleared here for k_rank_factor and k_rank_scale, which run after
};

// The value of a per-rank register array at rank k (lane k % 64, slot k / 64), on every lane; k is the same on all.
// Every slot is read from the lane, then the slot chosen, so the array is never indexed by a variable (which would
// put it in scratch memory).
template <int M>
__device__ __forceinline__ double rank_value(const double (&v)[M], uint32_t k) {
    if (k < 64) return readlane_f64(v[0], k);  // the truncation level's rows, most often
    double x = readlane_f64(v[0], k & 63u);
#pragma unroll
    for (int m = 1; m < M; ++m) {
        const double y = readlane_f64(v[m], k & 63u);
        x = static_cast<uint32_t>(m) == (k >> 6) ? y : x;
    }
    return x;
}
template <int M>
__device__ __forceinline__ float rank_value(const float (&v)[M], uint32_t k) {
    if (k < 64) return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[0]), k));
    float x = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[0]), k & 63u));
#pragma unroll
    for (int m = 1; m < M; ++m) {
        const float y = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v[m]), k & 63u));
        x = static_cast<uint32_t>(m) == (k >> 6) ? y : x;
    }
    return x;
}

// A query of at most NMAX rows on one wave (64 threads). NMAX: a power of two, 64..512. Lane l keeps ranks l + 64 m
// in registers: the row, score, label, gain and discount, and the rank's lambda and hessian sums.
template <int NMAX>
__global__ __launch_bounds__(64) void k_rank_pairs(RankArgs a) {
    constexpr int M = NMAX / 64;
    constexpr uint32_t STRIDE = NMAX + 4;  // the three term lists 32 bytes apart in the banks
    __shared__ __align__(16) double lds[3 * STRIDE];  // the sort's keys, then row i's terms in j order
    uint64_t *keys = reinterpret_cast<uint64_t *>(lds);
    const uint32_t q = a.queries[blockIdx.x], lane = threadIdx.x;
    if (a.flag && blockIdx.x == 0 && lane == 0) *a.flag = 0u;
    const uint32_t b = a.bounds[q], n = a.bounds[q + 1] - b;
    if (n == 0) {
        if (lane == 0) a.qsum[q] = 0.0;
        return;
    }
    // rank by score, descending, ties by row (lambdarank.rs:142-170): ascending (key, row), over the power of two
    // at or above n (at least 2), the keys past n sorting last
    const uint32_t span = n <= 2 ? 2u : 1u << (32 - __builtin_clz(n - 1));
    for (uint32_t k = lane; k < span; k += 64)
        keys[k] = k < n ? (static_cast<uint64_t>(srocm_rank::rank_key(a.scores[b + k])) << 32) | k : ~0ull;
    __syncthreads();
    for (uint32_t size = 2; size <= span; size <<= 1) {
        for (uint32_t half = size >> 1; half > 0; half >>= 1) {
            for (uint32_t t = lane; t < span; t += 64) {
                const uint32_t o = t ^ half;
                if (o > t) {
                    const uint64_t x = keys[t], y = keys[o];
                    if ((x > y) == ((t & size) == 0)) {
                        keys[t] = y;
                        keys[o] = x;
                    }
                }
            }
            __syncthreads();
        }
    }
    uint32_t row[M];
    double sc[M], gn[M], dc[M];
    float lb[M];
    uint32_t first_inf = n;  // the first rank with a -inf score: pairs stop there (lambdarank.rs:333-340)
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const uint32_t k = lane + 64u * m;
        row[m] = 0;
        sc[m] = gn[m] = dc[m] = 0.0;
        lb[m] = 0.0f;
        if (k < n) {
            const uint32_t r = static_cast<uint32_t>(keys[k] & 0xffffffffu);
            row[m] = r;
            sc[m] = static_cast<double>(a.scores[b + r]);
            lb[m] = a.label[b + r];
            gn[m] = a.label_gain[srocm_rank::label_as_index(lb[m])];
            dc[m] = a.discount[k];
            if (sc[m] == -__builtin_inf() && k < first_inf) first_inf = k;
        }
    }
    for (int o = 32; o > 0; o >>= 1) first_inf = min(first_inf, static_cast<uint32_t>(__shfl_xor(static_cast<int>(first_inf), o)));
    __syncthreads();  // the keys are read: the LDS holds the terms from here on
    const uint32_t valid = first_inf;
    uint32_t worst = n - 1;
    if (worst > 0 && rank_value(sc, worst) == -__builtin_inf()) --worst;
    const bool by_distance = a.norm && rank_value(sc, 0) != rank_value(sc, worst);
    const uint32_t rows_i = min(a.truncation, valid > 0 ? valid - 1 : 0u);
    const double inv_max_dcg = a.inv_max_dcg[q];
    double lam[M], hes[M];
#pragma unroll
    for (int m = 0; m < M; ++m) lam[m] = hes[m] = 0.0;
    double acc = 0.0;  // lane 2: the query's lambda sum

    // Row i's pairs the host takes (j > i, below the first -inf score, a different label): the ballot of each slot,
    // and each taken lane's arithmetic up to the table read. Step i starts row i (its table reads stay in flight) and
    // adds up row i - 1, whose terms step i - 1 listed.
    uint64_t take[M];
    double sign[M], ndcg[M], prob[M];
    uint32_t count = 0;  // row i - 1's taken pairs
    for (uint32_t i = 0; i <= rows_i; ++i) {
        double own_lam = 0.0, own_hes = 0.0;
        if (i > 0) {
            // row i - 1's terms: lane j adds its own to rank j's sums and lists it at its place among the row's
            // taken pairs
            count = 0;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if ((take[m] >> lane) & 1ull) {
                    srocm_rank::PairPrep pp;
                    pp.sign = sign[m];
                    pp.delta_ndcg = ndcg[m];
                    const srocm_rank::PairTerm t = srocm_rank::pair_finish(pp, prob[m], a.sigmoid, a.sigmoid2);
                    const double tl = t.sign * t.p_lambda, th = t.p_hessian;
                    lam[m] -= tl;
                    hes[m] += th;
                    const uint32_t at = count + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(take[m] >> 32),
                                                                          __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(take[m]), 0u));
                    lds[at] = tl;
                    lds[STRIDE + at] = th;
                    lds[2 * STRIDE + at] = -(2.0 * t.p_lambda);
                }
                count += static_cast<uint32_t>(__builtin_popcountll(take[m]));
            }
            __syncthreads();
            own_lam = rank_value(lam, i - 1);
            own_hes = rank_value(hes, i - 1);
        }
        if (i < rows_i) {
            const double si = rank_value(sc, i), gi = rank_value(gn, i), di = rank_value(dc, i);
            const float li = rank_value(lb, i);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint32_t j = lane + 64u * m;
                take[m] = 64u * m < valid ? __ballot(j > i && j < valid && lb[m] != li) : 0ull;
                if ((take[m] >> lane) & 1ull) {
                    const srocm_rank::PairPrep pp = srocm_rank::pair_prep(si, li, gi, di, sc[m], lb[m], gn[m], dc[m],
                                                                          inv_max_dcg, by_distance, a.min_input,
                                                                          a.max_input, a.idx_factor);
                    sign[m] = pp.sign;
                    ndcg[m] = pp.delta_ndcg;
                    prob[m] = a.table[pp.bin];
                }
            }
        }
        if (i > 0 && count > 0) {
            // row i - 1's own sums (from its sums as a lower rank) and the query's lambda sum, the terms in j order,
            // on lanes 0-2
            double s = lane == 0 ? own_lam : (lane == 1 ? own_hes : acc);
            if (lane < 3) {
                const double *src = lds + lane * STRIDE;
                uint32_t k = 0;
                for (; k + 8 <= count; k += 8) {
                    const double2 x0 = *reinterpret_cast<const double2 *>(src + k);
                    const double2 x1 = *reinterpret_cast<const double2 *>(src + k + 2);
                    const double2 x2 = *reinterpret_cast<const double2 *>(src + k + 4);
                    const double2 x3 = *reinterpret_cast<const double2 *>(src + k + 6);
                    s += x0.x;
                    s += x0.y;
                    s += x1.x;
                    s += x1.y;
                    s += x2.x;
                    s += x2.y;
                    s += x3.x;
                    s += x3.y;
                }
                for (; k < count; ++k) s += src[k];
                if (lane == 2) acc = s;
            }
            const double new_lam = readlane_f64(s, 0), new_hes = readlane_f64(s, 1);
            const uint32_t r = i - 1;
#pragma unroll
            for (int m = 0; m < M; ++m)
                if (static_cast<uint32_t>(m) == (r >> 6) && lane == (r & 63u)) {
                    lam[m] = new_lam;
                    hes[m] = new_hes;
                }
        }
        if (i > 0) __syncthreads();  // the term lists are rewritten for the next row
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const uint32_t k = lane + 64u * m;
        if (k < n) {
            a.lam[b + row[m]] = lam[m];
            a.hes[b + row[m]] = hes[m];
        }
    }
    if (lane == 2) a.qsum[q] = acc;
}

// The normalization factors' modes: 1 without normalization (RANK_FACTOR_ONE), the host's (RANK_FACTOR_HOST, made
// with the C library's log2 on the host), or made on the device from the lambda sums (RANK_FACTOR_DEVICE; and
// RANK_FACTOR_DEVICE_CHECKED, which flags every query: a host-forced test of the fallback).
constexpr uint32_t RANK_FACTOR_ONE = 0, RANK_FACTOR_HOST = 1, RANK_FACTOR_DEVICE = 2, RANK_FACTOR_DEVICE_CHECKED = 3;

// The device's factors of the `nq` listed queries, a thread each (norm_factor: log2(1 + s) / s for a lambda sum
// s > 0, else 1): pair[2q] from the round-down end of the log2 bracket, pair[2q + 1] from the round-up end (the same
// when log2(1 + s) is a double). An undecided bracket, or the checked mode, sets *flag.
__global__ __launch_bounds__(256) void k_rank_factor(const uint32_t *__restrict__ queries, uint32_t nq,
                                                     const double *__restrict__ qsum, uint32_t mode,
                                                     double *__restrict__ pair, uint32_t *__restrict__ flag) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    bool unsure = false;
    if (i < nq) {
        const uint32_t q = queries[i];
        const double s = qsum[q];
        double f0 = 1.0, f1 = 1.0;
        if (s > 0.0) {
            double lo, hi;
            const int st = srocm_log2::log2_bracket(1.0 + s, lo, hi);
            f0 = lo / s;
            f1 = hi / s;
            unsure = st == 2 || mode == RANK_FACTOR_DEVICE_CHECKED;
        }
        pair[2 * static_cast<size_t>(q)] = f0;
        pair[2 * static_cast<size_t>(q) + 1] = f1;
    }
    if (__ballot(unsure) && (threadIdx.x & 63u) == 0) atomicOr(flag, 1u);
}

// The gradients from the sums (lambdarank.rs:287-300, 405-415): g = f32(lambda * factor), h = f32(hessian *
// factor), each times the row's weight; the factor is the query's in `mode`: 1, the host's (`factor`), or the
// device's pair (`pair`, k_rank_factor), where a row whose f32 gradient or hessian differs between the pair's two
// factors sets *flag (the rows keep the first factor's values, and the host takes the iteration again with its own
// factors). A block (one wave) per query.
__global__ __launch_bounds__(64) void k_rank_scale(const uint32_t *__restrict__ bounds, const uint32_t *__restrict__ queries,
                                                   const double *__restrict__ lam, const double *__restrict__ hes,
                                                   const double *__restrict__ factor, const double *__restrict__ pair,
                                                   uint32_t mode, const float *__restrict__ weight, float *__restrict__ grad,
                                                   float *__restrict__ hess, uint32_t *__restrict__ flag) {
    const uint32_t q = queries[blockIdx.x], b = bounds[q], e = bounds[q + 1];
    double f0 = 1.0, f1 = 1.0;
    if (mode == RANK_FACTOR_HOST) {
        f0 = f1 = factor[q];
    } else if (mode >= RANK_FACTOR_DEVICE) {
        f0 = pair[2 * static_cast<size_t>(q)];
        f1 = pair[2 * static_cast<size_t>(q) + 1];
    }
    bool unsure = false;
    for (uint32_t r = b + threadIdx.x; r < e; r += 64) {
        float g = static_cast<float>(lam[r] * f0);
        float h = static_cast<float>(hes[r] * f0);
        if (f1 != f0)
            unsure = unsure || static_cast<float>(lam[r] * f1) != g || static_cast<float>(hes[r] * f1) != h;
        if (weight) {
            g *= weight[r];
            h *= weight[r];
        }
        grad[r] = g;
        hess[r] = h;
    }
    if (__ballot(unsure) && threadIdx.x == 0) atomicOr(flag, 1u);
}

}  // namespace srocm
