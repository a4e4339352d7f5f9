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

// max |v| over v as the bits of a non-negative float (order-preserving as unsigned), NaN skipped.
__device__ __forceinline__ void block_max_abs(float v, uint32_t *out) {
    float a = __builtin_fabsf(v);
    uint32_t bits = (a != a) ? 0u : __float_as_uint(a);
    for (int o = 32; o >= 1; o >>= 1) {
        uint32_t other = __shfl_xor(bits, o);
        bits = bits > other ? bits : other;
    }
    if ((threadIdx.x & 63) == 0) atomicMax(out, bits);
}

__global__ void k_grad_regression(const float *__restrict__ scores, const float *__restrict__ label,
                                  const float *__restrict__ weight, float *__restrict__ grad, float *__restrict__ hess,
                                  uint64_t n, uint32_t *maxima) {
    for (uint64_t base = blockIdx.x * (uint64_t)blockDim.x; base < n; base += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t r = base + threadIdx.x;
        float g = 0.0f, h = 0.0f;
        if (r < n) {
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
        }
        block_max_abs(g, maxima);
        block_max_abs(h, maxima + 1);
    }
}

// objective/binary.rs:27-50: f64 logloss gradients with an exp equal to the C library's, stored as f32
__global__ void k_grad_binary(const float *__restrict__ scores, const float *__restrict__ label,
                              const float *__restrict__ weight, float *__restrict__ grad, float *__restrict__ hess,
                              uint64_t n, double sigmoid, uint32_t *maxima) {
    for (uint64_t base = blockIdx.x * (uint64_t)blockDim.x; base < n; base += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t r = base + threadIdx.x;
        float g = 0.0f, h = 0.0f;
        if (r < n) {
            double sign = label[r] > 0.0f ? 1.0 : -1.0;
            double response = -sign * sigmoid / (1.0 + srocm_exp::exp(sign * sigmoid * static_cast<double>(scores[r])));
            double abs_response = __builtin_fabs(response);
            double w = weight ? static_cast<double>(weight[r]) : 1.0;
            g = static_cast<float>(response * w);
            h = static_cast<float>(abs_response * (sigmoid - abs_response) * w);
            grad[r] = g;
            hess[r] = h;
        }
        block_max_abs(g, maxima);
        block_max_abs(h, maxima + 1);
    }
}

__global__ void k_max_abs(const float *__restrict__ grad, const float *__restrict__ hess, uint64_t n, uint32_t *maxima) {
    for (uint64_t base = blockIdx.x * (uint64_t)blockDim.x; base < n; base += (uint64_t)gridDim.x * blockDim.x) {
        uint64_t r = base + threadIdx.x;
        block_max_abs(r < n ? grad[r] : 0.0f, maxima);
        block_max_abs(r < n ? hess[r] : 0.0f, maxima + 1);
    }
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
};

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

    uint32_t lb, n;
    leaf_rows(a.dev_left, a.begin, a.count, a.side, lb, n);
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
    const uint32_t *rows = a.rows + lb;
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
};

__global__ void k_hist_reduce(ReduceArgs a) {
    uint32_t lb, n;
    leaf_rows(a.dev_left, a.begin, a.count, a.side, lb, n);
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
    uint32_t per_block;    // rows per block (multiple of 256)
    // bagging
    uint32_t bag_seed, bag_round;
    uint64_t row_offset;
    double fraction;
};

__device__ __forceinline__ bool part_left(const PartArgs &a, uint32_t row) {
    if (a.col) {
        uint32_t bin = a.col[row];
        return (a.left_bins[bin >> 5] >> (bin & 31u)) & 1u;
    }
    return static_cast<double>(uniform(a.bag_seed, 2u, a.bag_round, a.row_offset + row)) < a.fraction;
}

__global__ __launch_bounds__(256) void k_part_count(PartArgs a) {
    __shared__ uint32_t wsum[4];
    uint32_t start = blockIdx.x * a.per_block;
    uint32_t end = start + a.per_block < a.count ? start + a.per_block : a.count;
    uint32_t c = 0;
    for (uint32_t i = start + threadIdx.x; i < end; i += 256) c += part_left(a, a.src[a.begin + i]) ? 1u : 0u;
    for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) a.block_left[blockIdx.x] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

__global__ __launch_bounds__(256) void k_part_scatter(PartArgs a) {
    __shared__ uint32_t red[2][4];
    __shared__ uint32_t wl[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    // lefts before this block, and in total
    uint32_t before = 0, total = 0;
    for (uint32_t j = tid; j < gridDim.x; j += 256) {
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
    uint32_t start = blockIdx.x * a.per_block;
    uint32_t end = start + a.per_block < a.count ? start + a.per_block : a.count;
    uint32_t lpos = before;                    // next left slot (relative to begin)
    uint32_t rpos = total + (start - before);  // next right slot
    for (uint32_t tile = start; tile < end; tile += 256) {
        uint32_t i = tile + tid;
        bool ok = i < end;
        uint32_t row = ok ? a.src[a.begin + i] : 0u;
        bool left = ok && part_left(a, row);
        uint64_t mask = __ballot(left);
        uint64_t valid = __ballot(ok);
        uint32_t below = __popcll(mask & ((1ull << lane) - 1ull));
        uint32_t below_valid = __popcll(valid & ((1ull << lane) - 1ull));
        if (lane == 0) wl[wave] = static_cast<uint32_t>(__popcll(mask));
        __syncthreads();
        uint32_t lbefore = 0, tile_left = 0;
        for (uint32_t w = 0; w < 4; ++w) {
            if (w < wave) lbefore += wl[w];
            tile_left += wl[w];
        }
        uint32_t tile_valid = (end - tile) < 256u ? (end - tile) : 256u;
        if (ok) {
            uint32_t idx_in_tile = wave * 64 + below_valid;  // == tid for valid lanes
            if (left) {
                a.dst[a.begin + lpos + lbefore + below] = row;
            } else {
                uint32_t rank = idx_in_tile - (lbefore + below);
                a.dst[a.begin + rpos + rank] = row;
            }
        }
        lpos += tile_left;
        rpos += tile_valid - tile_left;
        __syncthreads();
    }
}

__global__ void k_copy_u32(const uint32_t *__restrict__ src, uint32_t *__restrict__ dst, uint32_t begin, uint32_t n) {
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
__global__ __launch_bounds__(256) void k_split_scan(const ScanJob *__restrict__ jobs, const FeatDev *__restrict__ feats,
                                                    const uint8_t *__restrict__ evaluate, uint32_t num_features,
                                                    SplitCfgDev cfg, double sg, double sh) {
    const ScanJob &job = jobs[blockIdx.y];
    uint32_t f = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (f >= num_features) return;
    const int lane = threadIdx.x & 63;
    FeatCand r = {};
    FeatDev m = feats[f];
    Ctx c = make_ctx(cfg, sg, sh, job.units_grad, job.units_hess, job.count);
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

__global__ __launch_bounds__(256) void k_split_select(const ScanJob *__restrict__ jobs, uint32_t num_features,
                                                      SplitCfgDev cfg, double sg, double sh, SplitOut *out,
                                                      uint8_t *splittable /* [job][num_features] */) {
    const ScanJob &job = jobs[blockIdx.x];
    __shared__ double sgain[256];
    __shared__ int sfeat[256];
    double best = 0.0;
    int bf = -1;
    for (uint32_t f = threadIdx.x; f < num_features; f += 256) {
        const FeatCand &c = job.out[f];
        splittable[(size_t)blockIdx.x * num_features + f] = static_cast<uint8_t>(c.splittable);
        if (!c.found) continue;
        double g = (c.gain != c.gain) ? -__builtin_inf() : c.gain;
        if (bf < 0 || g > best) {  // features ascend within a thread, so ties keep the lower one
            best = g;
            bf = static_cast<int>(f);
        }
    }
    sgain[threadIdx.x] = best;
    sfeat[threadIdx.x] = bf;
    __syncthreads();
    for (int s = 128; s >= 1; s >>= 1) {
        if (threadIdx.x < s) {
            int fa = sfeat[threadIdx.x], fb = sfeat[threadIdx.x + s];
            double ga = sgain[threadIdx.x], gb = sgain[threadIdx.x + s];
            bool take_b = fb >= 0 && (fa < 0 || gb > ga || (gb == ga && fb < fa));
            if (take_b) {
                sgain[threadIdx.x] = gb;
                sfeat[threadIdx.x] = fb;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x != 0) return;
    SplitOut o = {};
    int f = sfeat[0];
    if (f >= 0) {
        const FeatCand &c = job.out[f];
        Ctx x = make_ctx(cfg, sg, sh, job.units_grad, job.units_hess, job.count);
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
    out[blockIdx.x] = o;
}

}  // namespace srocm
