// rank_kernels.hpp - LambdaRank-NDCG gradients on the device, bit for bit the host's f64 ones (lambdarank.hpp,
// which follows crates/silvic-core/src/objective/lambdarank.rs:190-420).
//
// One wave per query (k_rank_pairs): the query's rows are ranked by score (descending, ties by row) with a bitonic
// sort in LDS, then every row i above the truncation level takes its pairs (i, j), j > i, in order. The lanes compute
// the pair terms of row i for all j at once (the arithmetic is srocm_rank::pair_term, shared with the host), and lane
// j adds its own term to row j's sums, so each row's "as j" sums are taken over i in increasing order, as the host
// takes them. Row i's own sums and the query's lambda sum are running f64 sums in pair order; three lanes take them
// (lambda, hessian, lambda sum), each adding the terms of row i in j order, so every sum has the host's operation
// sequence. A pair the host skips (equal labels) contributes +0.0, which leaves a running sum unchanged: such a sum
// starts at +0.0 and never becomes -0.0 (x + (-x) rounds to +0.0), so x + 0.0 == x bit for bit.
//
// The unscaled sums go to per-row f64 buffers and the lambda sum to a per-query buffer. The normalization factor
// log2(1 + s) / s takes the host's log2 (one call per query, on the host, between k_rank_pairs and k_rank_scale), so
// the scaled f32 gradients equal the host's to the last bit.
#pragma once

#include "lambdarank.hpp"

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
};

// A query of at most NMAX rows on one wave (64 threads). NMAX: a power of two, 64..512.
template <int NMAX>
__global__ __launch_bounds__(64) void k_rank_pairs(RankArgs a) {
    constexpr int M = NMAX / 64;
    __shared__ uint64_t keys[NMAX];
    __shared__ double s_score[NMAX], s_gain[NMAX], s_disc[NMAX];
    __shared__ float s_lab[NMAX];
    __shared__ double terms[NMAX][3];  // row i's pair with rank j: lambda term, hessian term, -2 * p_lambda
    const uint32_t q = blockIdx.x, lane = threadIdx.x;
    const uint32_t b = a.bounds[q], n = a.bounds[q + 1] - b;
    if (n == 0) {
        if (lane == 0) a.qsum[q] = 0.0;
        return;
    }
    // rank by score, descending, ties by row (lambdarank.rs:142-170): ascending (key, row)
    for (uint32_t k = lane; k < NMAX; k += 64)
        keys[k] = k < n ? (static_cast<uint64_t>(srocm_rank::rank_key(a.scores[b + k])) << 32) | k : ~0ull;
    __syncthreads();
    for (uint32_t size = 2; size <= NMAX; size <<= 1) {
        for (uint32_t half = size >> 1; half > 0; half >>= 1) {
            for (uint32_t t = lane; t < NMAX; t += 64) {
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
    uint32_t first_inf = n;  // the first rank with a -inf score: pairs stop there (lambdarank.rs:333-340)
    for (uint32_t k = lane; k < n; k += 64) {
        const uint32_t r = static_cast<uint32_t>(keys[k] & 0xffffffffu);
        const double s = static_cast<double>(a.scores[b + r]);
        const float l = a.label[b + r];
        s_score[k] = s;
        s_lab[k] = l;
        s_gain[k] = a.label_gain[static_cast<uint32_t>(l)];
        s_disc[k] = a.discount[k];
        if (s == -__builtin_inf() && k < first_inf) first_inf = k;
    }
    for (int o = 32; o > 0; o >>= 1) first_inf = min(first_inf, static_cast<uint32_t>(__shfl_xor(static_cast<int>(first_inf), o)));
    __syncthreads();
    const uint32_t valid = first_inf;
    uint32_t worst = n - 1;
    if (worst > 0 && s_score[worst] == -__builtin_inf()) --worst;
    const bool by_distance = a.norm && s_score[0] != s_score[worst];
    const uint32_t rows_i = min(a.truncation, valid > 0 ? valid - 1 : 0u);
    const double inv_max_dcg = a.inv_max_dcg[q];
    double lam[M], hes[M];  // ranks lane + 64 m
#pragma unroll
    for (int m = 0; m < M; ++m) lam[m] = hes[m] = 0.0;
    double acc = 0.0;  // lane 2: the query's lambda sum
    for (uint32_t i = 0; i < rows_i; ++i) {
        const double si = s_score[i], gi = s_gain[i], di = s_disc[i];
        const float li = s_lab[i];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const uint32_t j = lane + 64u * m;
            double tl = 0.0, th = 0.0, tp = 0.0;
            if (j > i && j < valid && s_lab[j] != li) {
                const srocm_rank::PairTerm t =
                    srocm_rank::pair_term(si, li, gi, di, s_score[j], s_lab[j], s_gain[j], s_disc[j], inv_max_dcg,
                                          by_distance, a.sigmoid, a.sigmoid2, a.table, a.min_input, a.max_input,
                                          a.idx_factor);
                tl = t.sign * t.p_lambda;
                th = t.p_hessian;
                tp = -(2.0 * t.p_lambda);
                lam[m] -= tl;
                hes[m] += th;
            }
            if (j < NMAX) {
                terms[j][0] = tl;
                terms[j][1] = th;
                terms[j][2] = tp;
            }
        }
        __syncthreads();
        // row i's own sums (from its "as j" sums so far) and the query's lambda sum, in j order on lanes 0-2
        const uint32_t owner = i & 63u, mi = i >> 6;
        double li_lam = 0.0, li_hes = 0.0;
#pragma unroll
        for (int m = 0; m < M; ++m)
            if (static_cast<uint32_t>(m) == mi) {
                li_lam = lam[m];
                li_hes = hes[m];
            }
        li_lam = __shfl(li_lam, static_cast<int>(owner));
        li_hes = __shfl(li_hes, static_cast<int>(owner));
        if (lane < 3) {
            double s = lane == 0 ? li_lam : (lane == 1 ? li_hes : acc);
            uint32_t j = i + 1;
            for (; j + 4 <= valid; j += 4) {
                const double t0 = terms[j][lane], t1 = terms[j + 1][lane], t2 = terms[j + 2][lane], t3 = terms[j + 3][lane];
                s += t0;
                s += t1;
                s += t2;
                s += t3;
            }
            for (; j < valid; ++j) s += terms[j][lane];
            if (lane == 0) li_lam = s;
            else if (lane == 1) li_hes = s;
            else acc = s;
        }
        li_lam = __shfl(li_lam, 0);
        li_hes = __shfl(li_hes, 1);
#pragma unroll
        for (int m = 0; m < M; ++m)
            if (static_cast<uint32_t>(m) == mi && lane == owner) {
                lam[m] = li_lam;
                hes[m] = li_hes;
            }
        __syncthreads();  // the terms are rewritten for the next row
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const uint32_t k = lane + 64u * m;
        if (k < n) {
            const uint32_t r = static_cast<uint32_t>(keys[k] & 0xffffffffu);
            a.lam[b + r] = lam[m];
            a.hes[b + r] = hes[m];
        }
    }
    if (lane == 2) a.qsum[q] = acc;
}

// The gradients from the sums (lambdarank.rs:287-300, 405-415): g = f32(lambda * factor), h = f32(hessian *
// factor), each times the row's weight; the factor is the query's (1 without normalization). A block per query.
__global__ __launch_bounds__(64) void k_rank_scale(const uint32_t *__restrict__ bounds, const double *__restrict__ lam,
                                                   const double *__restrict__ hes, const double *__restrict__ factor,
                                                   const float *__restrict__ weight, float *__restrict__ grad,
                                                   float *__restrict__ hess) {
    const uint32_t q = blockIdx.x, b = bounds[q], e = bounds[q + 1];
    const double f = factor ? factor[q] : 1.0;
    for (uint32_t r = b + threadIdx.x; r < e; r += 64) {
        float g = static_cast<float>(lam[r] * f);
        float h = static_cast<float>(hes[r] * f);
        if (weight) {
            g *= weight[r];
            h *= weight[r];
        }
        grad[r] = g;
        hess[r] = h;
    }
}

}  // namespace srocm
