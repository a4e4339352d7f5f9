// kernels.hpp - gfx950 kernels of the quantized histogram / partition / split path.
//
// Compiled with -ffp-contract=off and without fast math: every f32/f64 operation below is the IEEE operation
// silvic's CPU path performs, in the same order, so quantized values and split decisions are bit-identical.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exp_f64.hpp"

namespace srocm {

constexpr double K_EPSILON = static_cast<double>(1e-15f);  // split.rs:37 (a float literal widened)
constexpr int WAVE = 64;

// ---------------------------------------------------------------------------------------------------------
// Rust numeric semantics on the device
// ---------------------------------------------------------------------------------------------------------

// `x as i32` for f32: truncation toward zero, saturating, NaN -> 0.
__device__ __forceinline__ int32_t sat_i32(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return 2147483647;
    if (x <= -2147483648.0f) return (-2147483647 - 1);
    return static_cast<int32_t>(x);
}

// `x as i64` for f64.
__device__ __forceinline__ int64_t sat_i64(double x) {
    if (x != x) return 0;
    if (x >= 9223372036854775807.0) return INT64_MAX;
    if (x <= -9223372036854775808.0) return INT64_MIN;
    return static_cast<int64_t>(x);
}

// f64::max (IEEE maxNum: a NaN operand yields the other).
__device__ __forceinline__ double max_num(double a, double b) {
    if (a != a) return b;
    if (b != b) return a;
    return a > b ? a : b;
}

// ---------------------------------------------------------------------------------------------------------
// quantize.rs:14-31 counter hash and quantize.rs:100-136 stochastic rounding
// ---------------------------------------------------------------------------------------------------------

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

__device__ __forceinline__ float uniform(uint32_t seed, uint32_t stream, uint32_t iteration, uint64_t row) {
    uint32_t row_hash = mix32(static_cast<uint32_t>(row) ^ mix32(static_cast<uint32_t>(row >> 32)));
    uint32_t h = mix32(seed ^ mix32(stream ^ mix32(iteration ^ row_hash)));
    return static_cast<float>(h >> 8) * (1.0f / 16777216.0f);
}

struct QuantDev {
    float inv_grad_scale, inv_hess_scale;
    int32_t grad_max_q, hess_max_q;
    uint32_t constant_hessian, stochastic, seed, iteration;
};

__device__ __forceinline__ int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

// quantize.rs:103-136 quantize_row
__device__ __forceinline__ int32_t quantize_row(const QuantDev &s, float grad, float hess, uint64_t row) {
    float q;
    if (s.stochastic) {
        float u = uniform(s.seed, 0u, s.iteration, row);
        q = grad >= 0.0f ? __builtin_truncf(__builtin_fmaf(grad, s.inv_grad_scale, u))
                         : __builtin_truncf(__builtin_fmaf(grad, s.inv_grad_scale, -u));
    } else {
        q = __builtin_rintf(grad * s.inv_grad_scale);
    }
    int32_t g = clamp_i32(sat_i32(q), -s.grad_max_q, s.grad_max_q);
    int32_t h;
    if (s.constant_hessian) {
        h = 1;
    } else {
        float p;
        if (s.stochastic) {
            float u = uniform(s.seed, 1u, s.iteration, row);
            p = __builtin_truncf(__builtin_fmaf(hess, s.inv_hess_scale, u));
        } else {
            p = __builtin_rintf(hess * s.inv_hess_scale);
        }
        h = clamp_i32(sat_i32(p), 0, s.hess_max_q);
    }
    return static_cast<int32_t>(static_cast<uint32_t>(h) * 65536u + static_cast<uint32_t>(g));
}

__global__ void k_quantize(const float *__restrict__ grad, const float *__restrict__ hess, int32_t *__restrict__ packed,
                           uint64_t n, uint64_t row_offset, QuantDev spec) {
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < n; r += (uint64_t)gridDim.x * blockDim.x)
        packed[r] = quantize_row(spec, grad[r], hess[r], row_offset + r);
}

// ---------------------------------------------------------------------------------------------------------
// gradients (objective/regression.rs:70-93: f32 arithmetic) and their maxima (cpu.rs:774)
// ---------------------------------------------------------------------------------------------------------

// max |v| as the bits of a non-negative float (order-preserving as unsigned), NaN skipped.
__device__ __forceinline__ uint32_t abs_bits(float v) {
    float a = __builtin_fabsf(v);
    return (a != a) ? 0u : __float_as_uint(a);
}

// Block-wide max of two per-thread values, one atomicMax each per block (blockDim 256).
__device__ __forceinline__ void block_max2(uint32_t a, uint32_t b, uint32_t *out) {
    __shared__ uint32_t sa[4], sb[4];
    for (int o = 32; o >= 1; o >>= 1) {
        uint32_t x = __shfl_xor(a, o), y = __shfl_xor(b, o);
        a = a > x ? a : x;
        b = b > y ? b : y;
    }
    if ((threadIdx.x & 63) == 0) {
        sa[threadIdx.x >> 6] = a;
        sb[threadIdx.x >> 6] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) {
            a = a > sa[w] ? a : sa[w];
            b = b > sb[w] ? b : sb[w];
        }
        atomicMax(out, a);
        atomicMax(out + 1, b);
    }
}

__global__ void k_grad_regression(const float *__restrict__ scores, const float *__restrict__ label,
                                  const float *__restrict__ weight, float *__restrict__ grad, float *__restrict__ hess,
                                  uint64_t n, uint32_t *maxima) {
    uint32_t mg = 0, mh = 0;
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < n; r += (uint64_t)gridDim.x * blockDim.x) {
        float g, h;
        float residual = scores[r] - label[r];
        if (weight) {
            g = residual * weight[r];
            h = weight[r];
        } else {
            g = residual;
            h = 1.0f;
        }
        grad[r] = g;
        hess[r] = h;
        uint32_t a = abs_bits(g), b = abs_bits(h);
        mg = mg > a ? mg : a;
        mh = mh > b ? mh : b;
    }
    block_max2(mg, mh, maxima);
}

// objective/binary.rs:27-50: f64 logloss gradients with an exp equal to the C library's, stored as f32
__global__ void k_grad_binary(const float *__restrict__ scores, const float *__restrict__ label,
                              const float *__restrict__ weight, float *__restrict__ grad, float *__restrict__ hess,
                              uint64_t n, double sigmoid, uint32_t *maxima) {
    uint32_t mg = 0, mh = 0;
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < n; r += (uint64_t)gridDim.x * blockDim.x) {
        double sign = label[r] > 0.0f ? 1.0 : -1.0;
        double response = -sign * sigmoid / (1.0 + srocm_exp::exp(sign * sigmoid * static_cast<double>(scores[r])));
        double abs_response = __builtin_fabs(response);
        double w = weight ? static_cast<double>(weight[r]) : 1.0;
        float g = static_cast<float>(response * w);
        float h = static_cast<float>(abs_response * (sigmoid - abs_response) * w);
        grad[r] = g;
        hess[r] = h;
        uint32_t a = abs_bits(g), b = abs_bits(h);
        mg = mg > a ? mg : a;
        mh = mh > b ? mh : b;
    }
    block_max2(mg, mh, maxima);
}

__global__ void k_max_abs(const float *__restrict__ grad, const float *__restrict__ hess, uint64_t n, uint32_t *maxima) {
    uint32_t mg = 0, mh = 0;
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < n; r += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t a = abs_bits(grad[r]), b = abs_bits(hess[r]);
        mg = mg > a ? mg : a;
        mh = mh > b ? mh : b;
    }
    block_max2(mg, mh, maxima);
}

__global__ void k_fill_f32(float *__restrict__ out, uint64_t n, float v) {
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < n; r += (uint64_t)gridDim.x * blockDim.x)
        out[r] = v;
}

__global__ void k_iota(uint32_t *__restrict__ out, uint64_t n) {
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < n; r += (uint64_t)gridDim.x * blockDim.x)
        out[r] = static_cast<uint32_t>(r);
}

// ---------------------------------------------------------------------------------------------------------
// Histogram of a leaf over one slab (a run of up to W features stored as W-byte rows).
//
// LDS holds the slab's histogram bin-major: word (bin * W + column), one packed i32 (h_q << 16) + g_q per bin
// (quantize.rs:100-107). A wave covers 64 / (W/4) rows, each lane one dword (4 columns) of a row. At step k a
// lane adds byte x = (k + (lane%32)/8) % 4 of its dword, so the 32 lanes of each half-wave hit the 32 LDS banks
// (bank = column mod 32 = 4 * (lane%8) + x) exactly once: every ds_add_u32 is conflict-free whatever the bins.
// Every `flush_rows` rows (<= 32767 / max_q, so no 16-bit half can overflow) the packed words are unpacked
// into per-thread registers (i32 g and h sums) and zeroed. Each workgroup writes its sums as a partial
// histogram `partial[wg][bin * W + column] = {g, h}`; k_hist_reduce adds the partials.
// ---------------------------------------------------------------------------------------------------------

// The split one step of a device-driven tree applies (learner.rs:249-352), written by the step before it and read
// by the step's partition, histogram and search kernels. `active` is 0 once the tree has stopped growing.
struct Plan {
    uint32_t active;          // this step splits a leaf
    uint32_t may_search;      // the children get a histogram and a split search (learner.rs:266-268)
    uint32_t index;           // the leaf split; it becomes the left child
    uint32_t begin, count;    // its rows in the partition
    uint32_t col;             // column-major index of the split feature
    uint32_t built_side;      // 0: the left child is histogrammed, 1: the right (learner.rs:271-275)
    int32_t parent_slot, built_slot;
    uint32_t left;            // rows going left, written by the partition
    uint32_t left_bins[8];
    int64_t parent_count;
    uint32_t used_columns;    // evaluated non-trivial features (the histogram's used columns)
    uint32_t src_buf;         // partition buffer holding the leaf's rows; its children go to the other one
};

struct HistArgs {
    const uint8_t *bins;      // slab rows: row r at bins + r * W
    const uint32_t *rows;     // partition buffer; the leaf's rows start at `begin`
    const int32_t *gh;        // packed quantized gradients per row
    int32_t *partial;         // [grid][256 * W][2]
    const uint32_t *dev_left; // when non-null: the leaf is the `side` child of [begin, begin+count) split at *dev_left
    uint32_t begin, count, side;
    uint32_t flush_rows;
    uint32_t max_groups;      // == gridDim.x
    uint32_t min_rows_per_group;
    const Plan *plan;         // when non-null, the leaf is the plan's built child (and nothing to do unless searched)
    const uint32_t *rows2;    // the second partition buffer, where a plan's children may live
};

// The leaf range of a histogram launch: from the plan when there is one. Returns false when there is nothing to do.
__device__ __forceinline__ bool hist_range(const Plan *plan, const uint32_t *dev_left, uint32_t begin, uint32_t count,
                                           uint32_t side, const uint32_t *&dl, uint32_t &b, uint32_t &c, uint32_t &s) {
    if (plan) {
        if (!plan->active || !plan->may_search) return false;
        dl = &plan->left;
        b = plan->begin;
        c = plan->count;
        s = plan->built_side;
    } else {
        dl = dev_left;
        b = begin;
        c = count;
        s = side;
    }
    return true;
}

// The rows of the leaf after resolving a device-side left count; identical in every kernel that calls it.
__device__ __forceinline__ void leaf_rows(const uint32_t *dev_left, uint32_t begin, uint32_t count, uint32_t side,
                                          uint32_t &b, uint32_t &n) {
    if (dev_left) {
        uint32_t left = *dev_left;
        if (side == 0) {
            b = begin;
            n = left;
        } else {
            b = begin + left;
            n = count - left;
        }
    } else {
        b = begin;
        n = count;
    }
}

// Workgroups used for n rows and rows per workgroup (a multiple of 64); identical in k_hist and k_hist_reduce.
__device__ __forceinline__ void hist_split(uint32_t n, uint32_t max_groups, uint32_t min_rows, uint32_t &groups,
                                           uint32_t &per) {
    uint32_t want = (n + min_rows - 1) / min_rows;
    groups = want < max_groups ? want : max_groups;
    if (groups == 0) groups = 1;
    per = (n + groups - 1) / groups;
    per = (per + 63u) & ~63u;
    if (per == 0) per = 64;
    groups = (n + per - 1) / per;
    if (groups == 0) groups = 1;
}

// Loads are branch-free: row positions past the range are clamped to its last row and their gradients
// zeroed, so the compiler issues every load of a step back to back instead of one masked load at a time. A
// wave fetches the row ids of its next step in one coalesced load (lane l: id l) while it works on the current
// step, and hands them out with a shuffle.
template <int W>
__global__ __launch_bounds__(1024) void k_hist(HistArgs a) {
    constexpr int DW = W / 4;                 // dwords per row
    constexpr int RPW = WAVE / DW;            // rows per wave step
    // row ids of one step fit one wave-wide load; at W = 128 the 64 accumulator registers leave room for 8
    constexpr int UNROLL = W == 128 ? 8 : (64 / RPW < 16 ? 64 / RPW : 16);
    constexpr uint32_t STEP = 16u * RPW * UNROLL;          // rows per block step (16 waves)
    constexpr int SLOTS = 256 * W / 1024;
    __shared__ int32_t lds[256 * W];

    const uint32_t *dl;
    uint32_t b0, c0, s0;
    if (!hist_range(a.plan, a.dev_left, a.begin, a.count, a.side, dl, b0, c0, s0)) return;
    uint32_t lb, n;
    leaf_rows(dl, b0, c0, s0, lb, n);
    uint32_t groups, per;
    hist_split(n, a.max_groups, a.min_rows_per_group, groups, per);
    if (blockIdx.x >= groups) return;
    const uint32_t tid = threadIdx.x;
    for (int j = 0; j < SLOTS; ++j) lds[tid + j * 1024] = 0;
    int32_t accg[SLOTS], acch[SLOTS];
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) accg[j] = acch[j] = 0;
    __syncthreads();

    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t d = lane % DW, rsub = lane / DW;
    const uint32_t rot = (lane & 31u) >> 3;
    const uint32_t *rows = (a.plan && !a.plan->src_buf ? a.rows2 : a.rows) + lb;
    const uint32_t *bins32 = reinterpret_cast<const uint32_t *>(a.bins);
    uint32_t start = blockIdx.x * per;
    uint32_t end = start + per < n ? start + per : n;

    for (uint32_t chunk = start; chunk < end; chunk += a.flush_rows) {
        uint32_t cend = chunk + a.flush_rows < end ? chunk + a.flush_rows : end;
        uint32_t last = cend - 1;
        uint32_t base = chunk + wave * RPW * UNROLL;
        uint32_t cidx = rows[min(base + lane, last)];
        for (; base < cend; base += STEP) {
            uint32_t r[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) r[u] = __shfl(cidx, u * RPW + rsub);
            cidx = rows[min(base + STEP + lane, last)];
            uint32_t dw[UNROLL];
            int32_t g[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                g[u] = a.gh[r[u]];
                dw[u] = bins32[(size_t)r[u] * DW + d];
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                int32_t gv = base + u * RPW + rsub < cend ? g[u] : 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    uint32_t x = (k + rot) & 3u;
                    uint32_t b = (dw[u] >> (8u * x)) & 255u;
                    atomicAdd(&lds[b * W + 4u * d + x], gv);
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < SLOTS; ++j) {
            int32_t v = lds[tid + j * 1024];
            lds[tid + j * 1024] = 0;
            int32_t gq = static_cast<int16_t>(static_cast<uint16_t>(static_cast<uint32_t>(v)));
            accg[j] += gq;
            acch[j] += (v - gq) >> 16;
        }
        __syncthreads();
    }
    int2 *out = reinterpret_cast<int2 *>(a.partial) + (size_t)blockIdx.x * (256 * W);
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) out[tid + j * 1024] = make_int2(accg[j], acch[j]);
}

// Adds the partials of one slab into the leaf histogram (i64 {g, h} per bin, flat layout). Thread per slab slot
// (bin * W + column); `col_offset[column]` is the column's feature's first bin in the flat histogram,
// `col_bins[column]` its bin count (0 for padding). When `parent` is non-null, also writes the sibling:
// sibling[bin] = parent[bin] - built[bin] (learner.rs:356-371), in place of the parent.
struct ReduceArgs {
    const int32_t *partial;
    const uint32_t *col_offset;
    const uint32_t *col_bins;
    int64_t *out;       // built child's histogram
    int64_t *parent;    // parent's histogram, overwritten with the sibling's (or null)
    const uint32_t *dev_left;
    uint32_t begin, count, side;
    uint32_t max_groups, min_rows_per_group;
    uint32_t width;     // W
    const Plan *plan;   // when non-null: out/parent are the plan's built/parent slots of `pool`
    int64_t *pool;
    uint64_t slot_stride;
};

__global__ void k_hist_reduce(ReduceArgs a) {
    const uint32_t *dl;
    uint32_t b0, c0, s0;
    if (!hist_range(a.plan, a.dev_left, a.begin, a.count, a.side, dl, b0, c0, s0)) return;
    if (a.plan) {
        a.out = a.pool + (size_t)a.plan->built_slot * a.slot_stride;
        a.parent = a.pool + (size_t)a.plan->parent_slot * a.slot_stride;
    }
    uint32_t lb, n;
    leaf_rows(dl, b0, c0, s0, lb, n);
    uint32_t groups, per;
    hist_split(n, a.max_groups, a.min_rows_per_group, groups, per);
    uint32_t slots = 256u * a.width;
    for (uint32_t s = blockIdx.x * blockDim.x + threadIdx.x; s < slots; s += gridDim.x * blockDim.x) {
        uint32_t col = s % a.width, bin = s / a.width;
        if (bin >= a.col_bins[col]) continue;
        int64_t g = 0, h = 0;
        const int2 *p = reinterpret_cast<const int2 *>(a.partial) + s;
        for (uint32_t w = 0; w < groups; ++w) {
            int2 v = p[(size_t)w * slots];
            g += v.x;
            h += v.y;
        }
        size_t o = 2 * ((size_t)a.col_offset[col] + bin);
        a.out[o] = g;
        a.out[o + 1] = h;
        if (a.parent) {
            a.parent[o] -= g;
            a.parent[o + 1] -= h;
        }
    }
}

// ---------------------------------------------------------------------------------------------------------
// Stable partition (cpu.rs:556-599) of a leaf's rows by a BinSplit, through a second buffer.
// Pass 1 counts each block's left rows; pass 2 recomputes every block's offset from those counts, compacts
// stably within the block (wave ballots + an LDS prefix over waves) and scatters; pass 3 copies back.
// Predicate: the bin of the split feature (column-major bins `col`) is set in `left_bins`; or, for bagging,
// quantize.rs:147-149 `in_bag` of the row.
// ---------------------------------------------------------------------------------------------------------

struct PartArgs {
    const uint32_t *src;   // rows
    uint32_t *dst;
    const uint8_t *col;    // column-major bins of the split feature (null: bagging predicate)
    uint32_t *block_left;  // [grid]
    uint32_t *dev_left;    // total left count (written by block 0 of pass 2)
    uint32_t begin, count;
    uint32_t left_bins[8];
    // bagging
    uint32_t bag_seed, bag_round;
    uint64_t row_offset;
    double fraction;
    Plan *plan;            // when non-null: range, split column and mask from the plan; the left count goes there
    const uint8_t *colbase;  // column-major bins of every feature ([feature][rows]) for the plan's column
    uint64_t rows;
    uint32_t *buf0, *buf1;   // the two partition buffers; the plan reads its leaf from one and writes the other
};

// Rows per block for `count` rows over the launch's blocks: a multiple of 256, the same in both passes.
__device__ __forceinline__ uint32_t part_per_block(uint32_t count, uint32_t blocks) {
    uint32_t per = (count + blocks - 1) / blocks;
    per = (per + 1023u) & ~1023u;
    return per < 1024u ? 1024u : per;
}

// Resolves the plan into the partition's range and predicate; false when the step does nothing.
__device__ __forceinline__ bool part_resolve(PartArgs &a) {
    if (!a.plan) return true;
    if (!a.plan->active) return false;
    a.begin = a.plan->begin;
    a.count = a.plan->count;
    a.src = a.plan->src_buf ? a.buf1 : a.buf0;
    a.dst = a.plan->src_buf ? a.buf0 : a.buf1;
    a.col = a.colbase + (size_t)a.plan->col * a.rows;
    a.dev_left = &a.plan->left;
    for (int i = 0; i < 8; ++i) a.left_bins[i] = a.plan->left_bins[i];
    return true;
}

__device__ __forceinline__ bool part_left(const PartArgs &a, uint32_t row) {
    if (a.col) {
        uint32_t bin = a.col[row];
        return (a.left_bins[bin >> 5] >> (bin & 31u)) & 1u;
    }
    return static_cast<double>(uniform(a.bag_seed, 2u, a.bag_round, a.row_offset + row)) < a.fraction;
}

// Tiles of 1024 rows: thread t takes rows t, t+256, t+512, t+768 of the tile (four sub-tiles of 256 in order),
// with every load of the tile issued before any is used (positions past the range are clamped and ignored).
__global__ __launch_bounds__(256) void k_part_count(PartArgs a) {
    __shared__ uint32_t wsum[4];
    if (!part_resolve(a)) return;
    const uint32_t per_block = part_per_block(a.count, gridDim.x);
    const uint32_t active = (a.count + per_block - 1) / per_block;
    if (blockIdx.x >= active && blockIdx.x > 0) return;
    const uint32_t start = blockIdx.x * per_block;
    const uint32_t end = start + per_block < a.count ? start + per_block : a.count;
    uint32_t c = 0;
    for (uint32_t tile = start; tile < end; tile += 1024) {
        uint32_t row[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) row[j] = a.src[a.begin + min(tile + j * 256 + threadIdx.x, end - 1)];
#pragma unroll
        for (int j = 0; j < 4; ++j) c += (tile + j * 256 + threadIdx.x < end && part_left(a, row[j])) ? 1u : 0u;
    }
    for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) a.block_left[blockIdx.x] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

__global__ __launch_bounds__(256) void k_part_scatter(PartArgs a) {
    __shared__ uint32_t red[2][4];
    __shared__ uint32_t wl[4][4];  // [sub-tile][wave] left counts
    if (!part_resolve(a)) return;
    const uint32_t per_block = part_per_block(a.count, gridDim.x);
    uint32_t active = (a.count + per_block - 1) / per_block;
    if (active == 0) active = 1;
    if (blockIdx.x >= active) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    // lefts before this block, and in total
    uint32_t before = 0, total = 0;
    for (uint32_t j = tid; j < active; j += 256) {
        uint32_t v = a.block_left[j];
        total += v;
        if (j < blockIdx.x) before += v;
    }
    for (int o = 32; o >= 1; o >>= 1) {
        before += __shfl_xor(before, o);
        total += __shfl_xor(total, o);
    }
    if (lane == 0) {
        red[0][wave] = before;
        red[1][wave] = total;
    }
    __syncthreads();
    before = red[0][0] + red[0][1] + red[0][2] + red[0][3];
    total = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    if (blockIdx.x == 0 && tid == 0 && a.dev_left) *a.dev_left = total;
    const uint32_t start = blockIdx.x * per_block;
    const uint32_t end = start + per_block < a.count ? start + per_block : a.count;
    uint32_t lpos = before;                    // next left slot (relative to begin)
    uint32_t rpos = total + (start - before);  // next right slot
    const uint64_t below_mask = (1ull << lane) - 1ull;
    for (uint32_t tile = start; tile < end; tile += 1024) {
        uint32_t row[4];
        bool ok[4], left[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t i = tile + j * 256 + tid;
            ok[j] = i < end;
            row[j] = a.src[a.begin + min(i, end - 1)];
        }
        uint32_t below[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            left[j] = ok[j] && part_left(a, row[j]);
            uint64_t m = __ballot(left[j]);
            below[j] = __popcll(m & below_mask);
            if (lane == 0) wl[j][wave] = static_cast<uint32_t>(__popcll(m));
        }
        __syncthreads();
        uint32_t lsub = 0;  // lefts in the sub-tiles before j
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t sub_start = tile + j * 256;
            uint32_t sub_valid = sub_start < end ? (end - sub_start < 256u ? end - sub_start : 256u) : 0u;
            uint32_t lbefore = 0, sub_left = 0;
            for (uint32_t w = 0; w < 4; ++w) {
                if (w < wave) lbefore += wl[j][w];
                sub_left += wl[j][w];
            }
            if (ok[j]) {
                uint32_t lrank = lsub + lbefore + below[j];  // lefts before this row in the tile
                if (left[j]) {
                    a.dst[a.begin + lpos + lrank] = row[j];
                } else {
                    uint32_t rrank = (sub_start - tile) + tid - lrank;  // rights before this row in the tile
                    a.dst[a.begin + rpos + rrank] = row[j];
                }
            }
            lsub += sub_left;
            (void)sub_valid;
        }
        uint32_t tile_valid = end - tile < 1024u ? end - tile : 1024u;
        lpos += lsub;
        rpos += tile_valid - lsub;
        __syncthreads();
    }
}

__global__ void k_copy_u32(const uint32_t *__restrict__ src, uint32_t *__restrict__ dst, uint32_t begin, uint32_t n,
                           const Plan *plan) {
    if (plan) {
        if (!plan->active) return;
        begin = plan->begin;
        n = plan->count;
    }
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        dst[begin + i] = src[begin + i];
}

// ---------------------------------------------------------------------------------------------------------
// leaf_sums (cpu.rs:886-908): exact fixed-point sums rint(v * scale) per leaf (quantize.rs:163-165)
// ---------------------------------------------------------------------------------------------------------

__device__ __forceinline__ int64_t to_fixed(float v, float scale) {
    float p = __builtin_rintf(v * scale);
    return sat_i64(static_cast<double>(p));
}

struct LeafJob {
    uint32_t begin, count, leaf;
};

__global__ __launch_bounds__(256) void k_leaf_sums(const float *__restrict__ grad, const float *__restrict__ hess,
                                                   const uint32_t *__restrict__ partition, const LeafJob *jobs,
                                                   float gs, float hs, unsigned long long *out, uint32_t chunk) {
    LeafJob j = jobs[blockIdx.y];
    uint32_t start = blockIdx.x * chunk;
    if (start >= j.count) return;
    uint32_t end = start + chunk < j.count ? start + chunk : j.count;
    int64_t sg = 0, sh = 0;
    for (uint32_t i = start + threadIdx.x; i < end; i += 256) {
        uint32_t r = partition[j.begin + i];
        sg += to_fixed(grad[r], gs);
        sh += to_fixed(hess[r], hs);
    }
    for (int o = 32; o >= 1; o >>= 1) {
        sg += __shfl_xor(sg, o);
        sh += __shfl_xor(sh, o);
    }
    if ((threadIdx.x & 63) == 0) {
        atomicAdd(out + 2 * j.leaf, static_cast<unsigned long long>(sg));
        atomicAdd(out + 2 * j.leaf + 1, static_cast<unsigned long long>(sh));
    }
}

// ---------------------------------------------------------------------------------------------------------
// add_tree (cpu.rs:666-695): walk each row down the tree on column-major bins, score += leaf value (f32)
// ---------------------------------------------------------------------------------------------------------

struct DevNode {
    uint32_t left_bins[8];
    uint32_t feature;  // index of the feature's column-major bins
    int32_t left, right;
    uint32_t pad;
};

__global__ void k_add_tree(const uint8_t *__restrict__ colbins, uint64_t rows, const DevNode *__restrict__ nodes,
                           const float *__restrict__ leaf_values, float *__restrict__ scores) {
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x) {
        int32_t node = 0;
        while (node >= 0) {
            const DevNode &nd = nodes[node];
            uint32_t bin = colbins[(size_t)nd.feature * rows + r];
            node = ((nd.left_bins[bin >> 5] >> (bin & 31u)) & 1u) ? nd.left : nd.right;
        }
        scores[r] += leaf_values[~node];
    }
}

__global__ void k_add_const(float *__restrict__ scores, uint64_t rows, float v) {
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x)
        scores[r] += v;
}

// ---------------------------------------------------------------------------------------------------------
// Best-split search (split.rs:201-961) for numerical features, one wave per (leaf, feature).
//
// A scan's running sums are sums of exact integers (quantized units and rounded per-bin counts), so a parallel
// prefix over the wave gives the same f64/i64 values as the reference's sequential loop. Every per-candidate
// value (hessians, constraints, the stopping candidate, gains) is then the same IEEE operation on the same
// operands; the best is the first maximum (NaN never wins), as ScanBuffer::best (split.rs:508-531).
// ---------------------------------------------------------------------------------------------------------

struct SplitCfgDev {
    int64_t min_data_in_leaf;
    double min_sum_hessian_in_leaf, lambda_l1, lambda_l2, min_gain_to_split;
};

struct Ctx {
    double units_grad, units_hess;
    int64_t num_data;
    double scale_grad, scale_hess;
    double sum_grad, sum_hess, cnt_factor, min_gain_shift;
    bool valid;
};

// split.rs:159-162
__device__ __forceinline__ double leaf_gain(double g, double h, double l1, double l2) {
    double r = max_num(__builtin_fabs(g) - l1, 0.0);
    return r * r / (h + l2);
}

// split.rs:145-154, 190-192
__device__ __forceinline__ double leaf_output(double g, double h, double l1, double l2) {
    double reg = max_num(__builtin_fabs(g) - l1, 0.0);
    double sign = static_cast<double>(static_cast<int>(g > 0.0) - static_cast<int>(g < 0.0));
    return -(sign * reg) / (h + l2);
}

// split.rs:214-233 LeafCtx::new
__device__ __forceinline__ Ctx make_ctx(const SplitCfgDev &cfg, double sg, double sh, double ug, double uh, int64_t count) {
    Ctx c;
    c.valid = !(uh != uh || uh <= 0.0 || count <= 0);
    c.units_grad = ug;
    c.units_hess = uh;
    c.num_data = count;
    c.scale_grad = sg;
    c.scale_hess = sh;
    c.sum_grad = ug * sg;
    c.sum_hess = uh * sh + 2.0 * K_EPSILON;
    double gain_shift = leaf_gain(c.sum_grad, c.sum_hess, cfg.lambda_l1, cfg.lambda_l2);
    c.cnt_factor = static_cast<double>(count) / c.sum_hess;
    c.min_gain_shift = gain_shift + cfg.min_gain_to_split;
    return c;
}

// A feature's best candidate (split.rs:298-317) as the search writes it per (leaf, feature).
struct FeatCand {
    int32_t found;        // a candidate exists
    int32_t splittable;   // any scan had a valid candidate
    double gain;          // best.gain - min_gain_shift
    double best_gain;     // the candidate's own split gain
    uint32_t threshold;
    uint32_t default_left;
    double left_grad, left_hess;
    int64_t left_count;
    double left_units_g, left_units_h;
};

struct Grown {
    uint32_t bin;
    double ug, uh;
    int64_t count;
    double gain;
};

// One scan direction over `n` bins of a feature's histogram slice `h` (i64 {g,h} pairs): element k is bin
// t0 + step * k. Lane l holds elements 4l..4l+3. Returns whether a candidate beat min_gain_shift.
__device__ bool wave_scan(const Ctx &c, const SplitCfgDev &cfg, const int64_t *h, int t0, int step, int n, Grown &out) {
    const int lane = threadIdx.x & 63;
    double pg[4], ph[4];
    int64_t pc[4];
    double lg = 0.0, lh = 0.0;
    int64_t lc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int k = 4 * lane + j;
        double gu = 0.0, hu = 0.0;
        int64_t ci = 0;
        if (k < n) {
            int t = t0 + step * k;
            gu = static_cast<double>(h[2 * t]);
            hu = static_cast<double>(h[2 * t + 1]);
            ci = sat_i64(hu * c.scale_hess * c.cnt_factor + 0.5);  // split.rs:196-198, 236-238
        }
        lg += gu;
        lh += hu;
        lc += ci;
        pg[j] = lg;
        ph[j] = lh;
        pc[j] = lc;
    }
    // exclusive prefix of the lane totals over the wave (exact: integer-valued)
    double eg = lg, eh = lh;
    int64_t ec = lc;
    for (int o = 1; o < 64; o <<= 1) {
        double ag = __shfl_up(eg, o);
        double ah = __shfl_up(eh, o);
        int64_t ac = __shfl_up(ec, o);
        if (lane >= o) {
            eg += ag;
            eh += ah;
            ec += ac;
        }
    }
    eg -= lg;
    eh -= lh;
    ec -= lc;
    const int64_t min_count = cfg.min_data_in_leaf > 1 ? cfg.min_data_in_leaf : 1;
    const double min_hess = cfg.min_sum_hessian_in_leaf;
    // split.rs:420-444: the first candidate where the other side is too small while the growing one is not
    int stop = n;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int k = 4 * lane + j;
        pg[j] += eg;
        ph[j] += eh;
        pc[j] += ec;
        if (k < n) {
            double hh = K_EPSILON + ph[j] * c.scale_hess;
            bool skip = pc[j] < min_count || hh < min_hess || ph[j] <= 0.0;
            bool other_small = c.num_data - pc[j] < min_count || c.sum_hess - hh < min_hess || c.units_hess - ph[j] <= 0.0;
            if (other_small && !skip && k < stop) stop = k;
        }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        int s = __shfl_xor(stop, o);
        stop = s < stop ? s : stop;
    }
    // split.rs:447-462 gains, split.rs:508-531 first maximum
    double gains[4];
    double m = -__builtin_inf();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int k = 4 * lane + j;
        gains[j] = -__builtin_inf();
        if (k < stop) {
            double hh = K_EPSILON + ph[j] * c.scale_hess;
            bool skip = pc[j] < min_count || hh < min_hess || ph[j] <= 0.0;
            double gg = pg[j] * c.scale_grad;
            double gain = leaf_gain(c.sum_grad - gg, c.sum_hess - hh, cfg.lambda_l1, cfg.lambda_l2) +
                          leaf_gain(gg, hh, cfg.lambda_l1, cfg.lambda_l2);
            gains[j] = skip ? -__builtin_inf() : gain;
            m = max_num(m, gains[j]);
        }
    }
    for (int o = 32; o >= 1; o >>= 1) m = max_num(m, __shfl_xor(m, o));
    if (!(m > c.min_gain_shift)) return false;
    int first = 1 << 30;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int k = 4 * lane + j;
        if (k < stop && gains[j] == m && k < first) first = k;
    }
    for (int o = 32; o >= 1; o >>= 1) {
        int s = __shfl_xor(first, o);
        first = s < first ? s : first;
    }
    int owner = first >> 2, jj = first & 3;
    double og = 0.0, oh = 0.0, ogain = 0.0;
    int64_t oc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (j == jj) {
            og = pg[j];
            oh = ph[j];
            oc = pc[j];
            ogain = gains[j];
        }
    out.ug = __shfl(og, owner);
    out.uh = __shfl(oh, owner);
    out.count = __shfl(oc, owner);
    out.gain = __shfl(ogain, owner);
    out.bin = static_cast<uint32_t>(t0 + step * first);
    return true;
}

struct FeatDev {
    uint32_t num_bins, hist_offset, kind, nan_bin;
};

struct ScanJob {
    const int64_t *hist;  // the leaf's histogram
    double units_grad, units_hess;
    int64_t count;
    FeatCand *out;        // [num_features]
};

// grid: (ceil(num_features / 4), num_jobs); 4 waves per block, a wave per feature.
// The exact row count of job `j`: the job's own, or the plan's child counts (left, then right).
__device__ __forceinline__ int64_t job_count(const ScanJob &job, const Plan *plan, uint32_t j) {
    if (!plan) return job.count;
    int64_t left = static_cast<int64_t>(plan->left);
    return j == 0 ? left : plan->parent_count - left;
}

__global__ __launch_bounds__(256) void k_split_scan(const ScanJob *__restrict__ jobs, const FeatDev *__restrict__ feats,
                                                    const uint8_t *__restrict__ evaluate, uint32_t num_features,
                                                    SplitCfgDev cfg, double sg, double sh, const Plan *plan) {
    if (plan && (!plan->active || !plan->may_search)) return;
    const ScanJob &job = jobs[blockIdx.y];
    uint32_t f = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (f >= num_features) return;
    const int lane = threadIdx.x & 63;
    FeatCand r = {};
    FeatDev m = feats[f];
    Ctx c = make_ctx(cfg, sg, sh, job.units_grad, job.units_hess, job_count(job, plan, blockIdx.y));
    if (c.valid && evaluate[f] && m.num_bins != 0 && m.kind == 1) {
        const int64_t *h = job.hist + 2 * static_cast<size_t>(m.hist_offset);
        int nb = static_cast<int>(m.num_bins);
        bool have = false;
        // split.rs:584-620 find_numerical
        if (m.nan_bin && nb > 2) {
            int last = nb - 2;
            Grown rg, fg;
            bool rf = wave_scan(c, cfg, h, last, -1, last, rg);
            bool ff = wave_scan(c, cfg, h, 0, 1, last + 1, fg);
            r.splittable = rf || ff;
            double output_gain = -__builtin_inf();
            if (rf) {  // split.rs:557-567 reverse_best
                double right_hess = K_EPSILON + rg.uh * c.scale_hess;
                r.best_gain = rg.gain;
                r.threshold = rg.bin - 1;
                r.left_grad = c.sum_grad - rg.ug * c.scale_grad;
                r.left_hess = c.sum_hess - right_hess;
                r.left_count = c.num_data - rg.count;
                r.left_units_g = c.units_grad - rg.ug;
                r.left_units_h = c.units_hess - rg.uh;
                r.default_left = 1;
                output_gain = rg.gain - c.min_gain_shift;
                have = true;
            }
            if (ff && fg.gain > output_gain + c.min_gain_shift) {  // split.rs:571-580 forward_best
                r.best_gain = fg.gain;
                r.threshold = fg.bin;
                r.left_grad = fg.ug * c.scale_grad;
                r.left_hess = K_EPSILON + fg.uh * c.scale_hess;
                r.left_count = fg.count;
                r.left_units_g = fg.ug;
                r.left_units_h = fg.uh;
                r.default_left = 0;
                have = true;
            }
        } else if (nb >= 2) {
            Grown rg;
            bool rf = wave_scan(c, cfg, h, nb - 1, -1, nb - 1, rg);
            r.splittable = rf;
            if (rf) {
                double right_hess = K_EPSILON + rg.uh * c.scale_hess;
                r.best_gain = rg.gain;
                r.threshold = rg.bin - 1;
                r.left_grad = c.sum_grad - rg.ug * c.scale_grad;
                r.left_hess = c.sum_hess - right_hess;
                r.left_count = c.num_data - rg.count;
                r.left_units_g = c.units_grad - rg.ug;
                r.left_units_h = c.units_hess - rg.uh;
                r.default_left = m.nan_bin ? 0 : 1;
                have = true;
            }
        }
        if (have) {
            r.found = 1;
            r.gain = r.best_gain - c.min_gain_shift;
        }
    }
    if (lane == 0) job.out[f] = r;
}

// The leaf's SplitInfo (split.rs:631-651 finish) and splittable flags from the per-feature candidates: the
// highest gain, NaN as -inf, ties to the lower feature (split.rs:866-880). One block per job.
struct SplitOut {
    int32_t found, feature;
    double gain;
    uint32_t threshold, default_left;
    double left_grad, left_hess;
    int64_t left_count;
    double right_grad, right_hess;
    int64_t right_count;
    double left_output, right_output;
};

// The best split over the per-feature candidates of `job` (highest gain, NaN as -inf, ties to the lower feature,
// split.rs:866-880) as the leaf's SplitOut (split.rs:631-651 finish), and its splittable flags. Block-wide (256).
// (gain, feature) order of split.rs:866-880 for reductions: a beats b on higher gain, then lower feature; -1 is
// "no candidate".
__device__ __forceinline__ bool cand_better(double ga, int fa, double gb, int fb) {
    return fa >= 0 && (fb < 0 || ga > gb || (ga == gb && fa < fb));
}

__device__ void select_split(const ScanJob &job, int64_t count, uint32_t num_features, const SplitCfgDev &cfg, double sg,
                             double sh, SplitOut *out, uint8_t *splittable) {
    __shared__ double wgain[4];
    __shared__ int wfeat[4];
    double best = 0.0;
    int bf = -1;
    for (uint32_t f = threadIdx.x; f < num_features; f += 256) {
        const FeatCand &c = job.out[f];
        splittable[f] = static_cast<uint8_t>(c.splittable);
        if (!c.found) continue;
        double g = (c.gain != c.gain) ? -__builtin_inf() : c.gain;
        if (cand_better(g, static_cast<int>(f), best, bf)) {
            best = g;
            bf = static_cast<int>(f);
        }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        double og = __shfl_xor(best, o);
        int of = __shfl_xor(bf, o);
        if (cand_better(og, of, best, bf)) {
            best = og;
            bf = of;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        wgain[threadIdx.x >> 6] = best;
        wfeat[threadIdx.x >> 6] = bf;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w)
            if (cand_better(wgain[w], wfeat[w], best, bf)) {
                best = wgain[w];
                bf = wfeat[w];
            }
        SplitOut o = {};
        int f = bf;
        if (f >= 0) {
            const FeatCand &c = job.out[f];
            Ctx x = make_ctx(cfg, sg, sh, job.units_grad, job.units_hess, count);
            o.found = 1;
            o.feature = f;
            o.gain = c.best_gain - x.min_gain_shift;
            o.threshold = c.threshold;
            o.default_left = c.default_left;
            o.left_grad = c.left_units_g;
            o.left_hess = c.left_units_h;
            o.left_count = c.left_count;
            o.right_grad = x.units_grad - c.left_units_g;
            o.right_hess = x.units_hess - c.left_units_h;
            o.right_count = x.num_data - c.left_count;
            o.left_output = leaf_output(c.left_grad, c.left_hess, cfg.lambda_l1, cfg.lambda_l2);
            o.right_output = leaf_output(x.sum_grad - c.left_grad, x.sum_hess - c.left_hess, cfg.lambda_l1, cfg.lambda_l2);
        }
        *out = o;
    }
    __syncthreads();
}

__global__ __launch_bounds__(256) void k_split_select(const ScanJob *__restrict__ jobs, uint32_t num_features,
                                                      SplitCfgDev cfg, double sg, double sh, SplitOut *out,
                                                      uint8_t *splittable /* [job][num_features] */) {
    const ScanJob &job = jobs[blockIdx.x];
    select_split(job, job.count, num_features, cfg, sg, sh, out + blockIdx.x, splittable + (size_t)blockIdx.x * num_features);
}

// ---------------------------------------------------------------------------------------------------------
// Device-driven growth (learner.rs:121-352): the leaf table, the tree arrays and the free list of histogram
// slots live on the device; each split step is partition -> histogram of the built child -> reduce + subtract
// -> split scan of both children -> k_apply, which updates the tree and the leaves and plans the next step.
// ---------------------------------------------------------------------------------------------------------

struct DLeaf {
    uint32_t begin, count;   // rows in the partition
    double ug, uh;           // sums in histogram units
    int64_t cnt;             // exact row count
    int32_t slot;            // histogram slot, -1: none
    uint32_t has_best;
    uint32_t buf;            // partition buffer holding the rows
    uint32_t pad_;
    SplitOut best;
};

struct TreeDev {
    int32_t *split_feature;
    uint32_t *threshold_bin;
    uint8_t *default_left;
    int32_t *left_child, *right_child;
    float *split_gain;
    double *internal_value, *internal_weight;
    int64_t *internal_count;
    double *leaf_value, *leaf_weight;
    int64_t *leaf_count;
    int32_t *leaf_parent, *leaf_depth;
};

struct GrowCtl {
    uint32_t num_leaves;     // the tree's leaves so far
    uint32_t done;           // no further split this tree
    uint32_t error;          // an invariant failed (a child without rows, no free histogram slot)
    int32_t free_top;        // entries on the free-slot stack
    double hist_rows;        // rows histogrammed (built children), and rows x evaluated features
    double hist_bins;
    double hist_builds;      // child histograms built
};

struct GrowState {
    GrowCtl *ctl;
    Plan *plan;
    DLeaf *leaves;
    uint8_t *splittable;     // [leaf][nf]
    int32_t *free_slots;
    ScanJob *jobs;           // [2]
    FeatCand *cands;         // [2][nf]
    uint8_t *evaluate;       // [nf]
    const uint8_t *mask;     // [nf], the tree's feature mask
    const FeatDev *feats;
    const int32_t *feat_nt;  // feature -> column-major index
    TreeDev tree;
    int64_t *pool;
    uint64_t slot_stride;
    uint32_t nf, num_leaves, sums_feature;
    int32_t max_depth;
    SplitCfgDev cfg;
    double sg, sh;
};

__device__ __forceinline__ bool depth_allows(const GrowState &g, int32_t d) { return g.max_depth <= 0 || d < g.max_depth; }

// learner.rs:418-429 best_leaf, then learner.rs:249-290: the next step's plan. Block-wide.
__device__ void plan_next(const GrowState &g) {
    __shared__ double bgain[4];
    __shared__ int bidx[4];
    GrowCtl *ctl = g.ctl;
    uint32_t n = ctl->num_leaves;
    bool stop = ctl->done || ctl->error || n >= g.num_leaves;
    double best = 0.0;
    int bi = -1;
    if (!stop)
        for (uint32_t i = threadIdx.x; i < n; i += 256) {  // leaves ascend within a thread: ties keep the first
            const DLeaf &l = g.leaves[i];
            if (!l.has_best) continue;
            if (bi < 0 || l.best.gain > best) {
                best = l.best.gain;
                bi = static_cast<int>(i);
            }
        }
    for (int o = 32; o >= 1; o >>= 1) {
        double og = __shfl_xor(best, o);
        int oi = __shfl_xor(bi, o);
        if (cand_better(og, oi, best, bi)) {
            best = og;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        bgain[threadIdx.x >> 6] = best;
        bidx[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < 4; ++w)
            if (cand_better(bgain[w], bidx[w], bgain[0], bidx[0])) {
                bgain[0] = bgain[w];
                bidx[0] = bidx[w];
            }
    __syncthreads();
    int index = bidx[0];
    bool go = !stop && index >= 0 && bgain[0] > 0.0;
    __syncthreads();
    if (!go) {
        if (threadIdx.x == 0) {
            g.plan->active = 0;
            ctl->done = 1;
        }
        return;
    }
    DLeaf &leaf = g.leaves[index];
    const SplitOut &info = leaf.best;
    __shared__ uint32_t used_w[4];
    uint32_t used = 0;
    for (uint32_t f = threadIdx.x; f < g.nf; f += 256) {
        uint8_t e = static_cast<uint8_t>(g.mask[f] && g.splittable[(size_t)index * g.nf + f]);
        g.evaluate[f] = e;
        used += (e && g.feats[f].num_bins) ? 1u : 0u;
    }
    for (int o = 32; o >= 1; o >>= 1) used += __shfl_xor(used, o);
    if ((threadIdx.x & 63) == 0) used_w[threadIdx.x >> 6] = used;
    __syncthreads();
    if (threadIdx.x == 0) {
        Plan &p = *g.plan;
        FeatDev m = g.feats[info.feature];
        p.active = 1;
        p.index = static_cast<uint32_t>(index);
        p.begin = leaf.begin;
        p.count = leaf.count;
        p.parent_count = leaf.cnt;
        p.src_buf = leaf.buf;
        p.col = static_cast<uint32_t>(g.feat_nt[info.feature]);
        // learner.rs:432-452: bins 0..=threshold, and the NaN bin when missing values go left
        uint32_t words[8];
        for (uint32_t w = 0; w < 8; ++w) {
            uint32_t lo = 32 * w;
            uint32_t upto = info.threshold + 1;  // bins below `upto` go left
            words[w] = upto >= lo + 32 ? 0xffffffffu : (upto > lo ? (1u << (upto - lo)) - 1u : 0u);
        }
        if (info.default_left && m.nan_bin) words[(m.num_bins - 1) >> 5] |= 1u << ((m.num_bins - 1) & 31u);
        for (uint32_t w = 0; w < 8; ++w) p.left_bins[w] = words[w];
        p.used_columns = used_w[0] + used_w[1] + used_w[2] + used_w[3];
        p.built_side = info.left_count <= info.right_count ? 0u : 1u;
        p.may_search = leaf.slot >= 0 && n + 1 < g.num_leaves && depth_allows(g, g.tree.leaf_depth[index] + 1);
        p.parent_slot = leaf.slot;
        p.built_slot = -1;
        if (p.may_search) {
            if (ctl->free_top <= 0) {
                ctl->error = 2;
                p.may_search = 0;
            } else {
                p.built_slot = g.free_slots[--ctl->free_top];
            }
        }
        if (p.may_search) {
            int64_t *built = g.pool + (size_t)p.built_slot * g.slot_stride;
            int64_t *parent = g.pool + (size_t)p.parent_slot * g.slot_stride;
            // jobs: the left child, then the right; their exact counts come from the partition
            g.jobs[0] = ScanJob{p.built_side == 0 ? built : parent, info.left_grad, info.left_hess, 0, g.cands};
            g.jobs[1] = ScanJob{p.built_side == 0 ? parent : built, info.right_grad, info.right_hess, 0, g.cands + g.nf};
        }
        leaf.has_best = 0;
    }
    __syncthreads();
}

// Copies the rows of every leaf that ended in the second partition buffer back into the first. grid: (x, leaves).
__global__ void k_consolidate(GrowState g, const uint32_t *__restrict__ buf1, uint32_t *__restrict__ buf0) {
    if (blockIdx.y >= g.ctl->num_leaves) return;
    const DLeaf &l = g.leaves[blockIdx.y];
    if (!l.buf) return;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < l.count; i += gridDim.x * blockDim.x)
        buf0[l.begin + i] = buf1[l.begin + i];
}

// The tree at its start: one leaf holding the root rows; slot 0 for its histogram when it is searched.
__global__ void k_grow_init(GrowState g, uint32_t root_begin, uint32_t root_count, int64_t root_cnt, uint32_t slots,
                            uint32_t searched) {
    for (uint32_t i = threadIdx.x; i < slots; i += blockDim.x) g.free_slots[i] = static_cast<int32_t>(slots - 1 - i);
    __syncthreads();
    if (threadIdx.x == 0) {
        GrowCtl &c = *g.ctl;
        c.num_leaves = 1;
        c.done = 0;
        c.error = 0;
        c.free_top = static_cast<int32_t>(slots);
        c.hist_rows = 0.0;
        c.hist_bins = 0.0;
        c.hist_builds = 0.0;
        g.plan->active = 0;
        DLeaf l = {};
        l.begin = root_begin;
        l.count = root_count;
        l.cnt = root_cnt;
        l.slot = searched ? g.free_slots[--c.free_top] : -1;
        g.leaves[0] = l;
        g.tree.leaf_value[0] = 0.0;
        g.tree.leaf_weight[0] = 0.0;
        g.tree.leaf_count[0] = 0;
        g.tree.leaf_parent[0] = -1;
        g.tree.leaf_depth[0] = 0;
    }
}

// learner.rs:143-156: the root's sums from the sums feature's bins (split.rs:101-108), and its search job.
__global__ void k_root_prep(GrowState g) {
    const DLeaf &l = g.leaves[0];
    const int64_t *h = g.pool + (size_t)l.slot * g.slot_stride;
    for (uint32_t f = threadIdx.x; f < g.nf; f += blockDim.x) g.evaluate[f] = g.mask[f];
    if (threadIdx.x == 0) {
        FeatDev m = g.feats[g.sums_feature];
        double sg = 0.0, sh = 0.0;
        for (uint32_t b = 0; b < m.num_bins; ++b) {
            sg = sg + static_cast<double>(h[2 * ((size_t)m.hist_offset + b)]);
            sh = sh + static_cast<double>(h[2 * ((size_t)m.hist_offset + b) + 1]);
        }
        g.leaves[0].ug = sg;
        g.leaves[0].uh = sh;
        g.jobs[0] = ScanJob{h, sg, sh, l.cnt, g.cands};
    }
}

__global__ __launch_bounds__(256) void k_root_select(GrowState g) {
    ScanJob job = g.jobs[0];
    __shared__ SplitOut o;
    select_split(job, job.count, g.nf, g.cfg, g.sg, g.sh, &o, g.splittable);
    if (threadIdx.x == 0) {
        g.leaves[0].best = o;
        g.leaves[0].has_best = o.found ? 1u : 0u;
    }
    __syncthreads();
    plan_next(g);
}

// learner.rs:294-352: apply the planned split with the exact left count, set up the children (their best splits
// when searched), free unused histogram slots, then plan the next step. One block.
__global__ __launch_bounds__(256) void k_apply(GrowState g) {
    const Plan &p = *g.plan;
    if (!p.active) return;
    __shared__ int searched;
    GrowCtl *ctl = g.ctl;
    const uint32_t index = p.index;
    const uint32_t new_leaf = ctl->num_leaves;
    const int64_t left = static_cast<int64_t>(p.left);
    const int64_t right = p.parent_count - left;
    if (threadIdx.x == 0) {
        const SplitOut info = g.leaves[index].best;
        searched = 0;
        if (left <= 0 || right <= 0) {
            ctl->error = 1;
        } else {
            // tree.rs:143-177 Tree::split
            const TreeDev &t = g.tree;
            int32_t node = static_cast<int32_t>(new_leaf) - 1;
            int32_t parent = t.leaf_parent[index];
            if (parent >= 0) {
                if (t.left_child[parent] == ~static_cast<int32_t>(index)) t.left_child[parent] = node;
                else t.right_child[parent] = node;
            }
            t.split_feature[node] = info.feature;
            t.split_gain[node] = static_cast<float>(info.gain + g.cfg.min_gain_to_split);
            t.threshold_bin[node] = info.threshold;
            t.default_left[node] = static_cast<uint8_t>(info.default_left);
            t.left_child[node] = ~static_cast<int32_t>(index);
            t.right_child[node] = ~static_cast<int32_t>(new_leaf);
            t.internal_weight[node] = t.leaf_weight[index];
            t.internal_value[node] = t.leaf_value[index];
            t.internal_count[node] = left + right;
            double lv = info.left_output, rv = info.right_output;
            t.leaf_value[index] = lv != lv ? 0.0 : lv;
            t.leaf_weight[index] = info.left_hess * g.sh;
            t.leaf_count[index] = left;
            t.leaf_value[new_leaf] = rv != rv ? 0.0 : rv;
            t.leaf_weight[new_leaf] = info.right_hess * g.sh;
            t.leaf_count[new_leaf] = right;
            t.leaf_parent[index] = node;
            t.leaf_parent[new_leaf] = node;
            int32_t depth = t.leaf_depth[index] + 1;
            t.leaf_depth[index] = depth;
            t.leaf_depth[new_leaf] = depth;
            // the children (learner.rs:320-334)
            DLeaf l = {}, r = {};
            l.begin = p.begin;
            l.count = p.left;
            l.ug = info.left_grad;
            l.uh = info.left_hess;
            l.cnt = left;
            l.slot = -1;
            l.buf = 1u - p.src_buf;
            r.buf = 1u - p.src_buf;
            r.begin = p.begin + p.left;
            r.count = p.count - p.left;
            r.ug = info.right_grad;
            r.uh = info.right_hess;
            r.cnt = right;
            r.slot = -1;
            int64_t min_pair = 2 * g.cfg.min_data_in_leaf;
            bool s = p.may_search && depth_allows(g, depth) && (left >= min_pair || right >= min_pair);
            if (p.may_search) {  // the built child's histogram was made, searched or not
                double built_rows = p.built_side == 0 ? static_cast<double>(left) : static_cast<double>(right);
                ctl->hist_rows += built_rows;
                ctl->hist_bins += built_rows * static_cast<double>(p.used_columns);
                ctl->hist_builds += 1.0;
            }
            if (s) {
                l.slot = p.built_side == 0 ? p.built_slot : p.parent_slot;
                r.slot = p.built_side == 0 ? p.parent_slot : p.built_slot;
            } else {
                if (p.parent_slot >= 0) g.free_slots[ctl->free_top++] = p.parent_slot;
                if (p.built_slot >= 0) g.free_slots[ctl->free_top++] = p.built_slot;
            }
            g.leaves[index] = l;
            g.leaves[new_leaf] = r;
            ctl->num_leaves = new_leaf + 1;
            searched = s ? 1 : 0;
        }
    }
    __syncthreads();
    if (searched) {
        __shared__ SplitOut o;
        for (uint32_t j = 0; j < 2; ++j) {
            ScanJob job = g.jobs[j];
            uint32_t who = j == 0 ? index : new_leaf;
            select_split(job, j == 0 ? left : right, g.nf, g.cfg, g.sg, g.sh, &o, g.splittable + (size_t)who * g.nf);
            if (threadIdx.x == 0) {
                g.leaves[who].best = o;
                g.leaves[who].has_best = o.found ? 1u : 0u;
            }
            __syncthreads();
        }
    }
    plan_next(g);
}

}  // namespace srocm
