// kernels.hpp - gfx950 kernels of the quantized histogram / partition / split path.
//
// Compiled with -ffp-contract=off and without fast math: every f32/f64 operation below is the IEEE operation
// silvic's CPU path performs, in the same order, so quantized values and split decisions are bit-identical.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "exp_f64.hpp"
#include "packed_word.hpp"

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

// The gradient maxima live in MAX_SLOTS pairs of words: block b adds its own to pair b mod MAX_SLOTS, so at most
// ceil(blocks / MAX_SLOTS) atomics meet at one address (atomics on one address are served one at a time, about
// 11 ns each: 2048 blocks on one pair took 49 us where the loads took 4), and readers take the largest pair-wise.
constexpr uint32_t MAX_SLOTS = 64;

// An iteration's quantization made on the device from the gradient maxima, so the boosting loop never waits for
// them: the scales of quantize.rs:56-84 and the fixed-point scales of quantize.rs:153-159, in the host's double
// operations (ceil(log2 x) from the exponent: exact for the float maxima these are).
struct DevScales {
    double sg, sh;    // grad_scale, hess_scale
    float gsc, hsc;   // the leaf sums' fixed-point scales
    QuantDev q;
};

__device__ __forceinline__ double positive_or_one_d(double v) { return v > 0.0 && __builtin_isfinite(v) ? v : 1.0; }

__device__ __forceinline__ float fixed_point_scale_d(double max_abs) {
    if (!__builtin_isfinite(max_abs) || max_abs <= 0.0) return 1.0f;
    int ex = 0;
    const double m = __builtin_frexp(max_abs, &ex);  // max_abs = m * 2^ex, m in [0.5, 1)
    int e = 30 - (m == 0.5 ? ex - 1 : ex);
    e = e < -126 ? -126 : (e > 127 ? 127 : e);
    return __builtin_ldexpf(1.0f, e);
}

// One wave (launched with MAX_SLOTS threads): lane l reads slot pair l of the maxima and clears it, so the next
// gradients' maxima start from zero without a fill of their own.
__global__ void k_quant_spec(uint32_t *maxima, DevScales *out, uint32_t num_bins, uint32_t constant_hessian,
                             double constant, uint32_t stochastic, uint32_t seed, uint32_t iteration) {
    uint32_t ug = maxima[2u * threadIdx.x], uh = maxima[2u * threadIdx.x + 1u];
    maxima[2u * threadIdx.x] = 0u;
    maxima[2u * threadIdx.x + 1u] = 0u;
    for (int o = 32; o >= 1; o >>= 1) {
        const uint32_t x = __shfl_xor(ug, o), y = __shfl_xor(uh, o);
        ug = ug > x ? ug : x;
        uh = uh > y ? uh : y;
    }
    static_assert(MAX_SLOTS == 64, "one slot pair a lane");
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const double mg = static_cast<double>(__uint_as_float(ug)), mh = static_cast<double>(__uint_as_float(uh));
    DevScales d;
    d.q.grad_max_q = static_cast<int32_t>(num_bins / 2);
    d.q.hess_max_q = static_cast<int32_t>(num_bins);
    d.sg = positive_or_one_d(mg / static_cast<double>(d.q.grad_max_q));
    d.sh = constant_hessian ? positive_or_one_d(constant) : positive_or_one_d(mh / static_cast<double>(d.q.hess_max_q));
    d.q.inv_grad_scale = static_cast<float>(1.0 / d.sg);
    d.q.inv_hess_scale = static_cast<float>(1.0 / d.sh);
    d.q.constant_hessian = constant_hessian;
    d.q.stochastic = stochastic;
    d.q.seed = seed;
    d.q.iteration = iteration;
    d.gsc = fixed_point_scale_d(mg);
    d.hsc = fixed_point_scale_d(mh);
    *out = d;
}

__global__ void k_quantize_dev(const float *__restrict__ grad, const float *__restrict__ hess, int32_t *__restrict__ packed,
                               uint64_t n, uint64_t row_offset, const DevScales *sc) {
    const QuantDev spec = sc->q;
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

// Block-wide max of two per-thread values, one atomicMax each per block into its slot pair (blockDim 256).
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
        uint32_t *slot = out + 2u * (blockIdx.x % MAX_SLOTS);
        atomicMax(slot, a);
        atomicMax(slot + 1, b);
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

__global__ void k_zero_i64(int64_t *__restrict__ out, uint64_t n) {
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < n; r += (uint64_t)gridDim.x * blockDim.x)
        out[r] = 0;
}

// Column-major bins, one byte per bin, or two (little-endian u16) when the dataset has features of more than 256
// bins (`col16`).
__device__ __forceinline__ uint32_t col_bin(const uint8_t *col, uint32_t col16, size_t i) {
    return col16 ? static_cast<uint32_t>(reinterpret_cast<const uint16_t *>(col)[i]) : static_cast<uint32_t>(col[i]);
}

// Whether a split sends `bin` left: a byte feature's split is its 256-bit mask (BinSplit::goes_left,
// backend/mod.rs:34-37); a feature of more than 256 bins (`wide`) carries its numerical rule in the words instead:
// lb[0] the threshold, lb[1] the NaN bin + 1 when missing values go left (0 otherwise).
__device__ __forceinline__ bool rule_left(const uint32_t *lb, uint32_t wide, uint32_t bin) {
    if (wide) return bin <= lb[0] || (lb[1] != 0u && bin == lb[1] - 1u);
    return ((lb[bin >> 5] >> (bin & 31u)) & 1u) != 0u;
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
// Every `flush_rows` rows (at most 32767 / max |g| and 65535 / max h: the low half holds g as a signed 16-bit
// value, the high half h, which is never negative, as an unsigned one) the packed words are unpacked into per-thread
// registers (i32 g and h sums) and zeroed. Each workgroup writes its sums as a partial
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
    const uint32_t *pos_word; // dense slab: per row byte, its LDS word at bin 0 (segment base * W + column)
    uint32_t dw_row;          // dense slab: dwords per row
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

// A lane's four adds per row dword, in the conflict-free order: at step k byte x = (k + rot) % 4, i.e. bits 8x..8x+7
// (xs[k] = 8x), is the row's byte i = 4d + x and goes to column i (cols[k]). In a packed slab (PACK features of at
// most 256 / PACK bins a column) byte i goes to column i % W, in the rows of its segment i / W: cols[k] is then
// the word offset of that segment's column, and a bin b adds to word b * W + cols[k] as in a byte slab (the bank
// is still the column's).
template <int W, int PACK>
__device__ __forceinline__ void row_bin_lanes(uint32_t d, uint32_t rot, uint32_t (&xs)[4], uint32_t (&cols)[4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t x = (k + rot) & 3u;
        const uint32_t i = 4u * d + x;
        xs[k] = 8u * x;
        cols[k] = PACK == 1 ? i : (i / W) * (256u / PACK) * W + i % W;
    }
}

// Adds gv to the LDS words (bin * W + column) of the four bins in a row dword: each bin is extracted in place (one
// bit-field extract) and scaled into its word address with the column added (one shift-add). Q32: the LDS holds
// separate 32-bit g and h counters (g words first, then 256 * W h words), and gv, hv are the row's g and h.
template <int W, int PACK = 1, bool Q32 = false>
__device__ __forceinline__ void add_row_bins(int32_t *lds, uint32_t dw, int32_t gv, int32_t hv, const uint32_t (&xs)[4],
                                             const uint32_t (&cols)[4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t b = __builtin_amdgcn_ubfe(dw, xs[k], 8u);
        if constexpr (PACK > 1) b &= 256u / PACK - 1u;  // a packed column's segment: invalid bins stay in it
        atomicAdd(&lds[b * W + cols[k]], gv);
        if constexpr (Q32) atomicAdd(&lds[256 * W + b * W + cols[k]], hv);
    }
}

// A wide slab (two-byte bins of up to 1024, W / 4 features) keeps the byte slab's LDS and partial shape: bin b of
// its column c is word (b >> 2) * W + (b & 3) * (W / 4) + c, i.e. a wide column is four virtual byte columns (bins
// congruent to 0, 1, 2, 3 mod 4). A lane's dword holds the bins of columns 2d and 2d + 1.
template <int W, bool Q32 = false>
__device__ __forceinline__ void add_row_bins_wide(int32_t *lds, uint32_t dw, int32_t gv, int32_t hv, uint32_t d) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const uint32_t b = min((dw >> (16 * k)) & 0xffffu, 1023u);  // clamped: invalid bins stay inside the LDS
        const uint32_t w = (b >> 2) * W + (b & 3u) * (W / 4) + 2u * d + k;
        atomicAdd(&lds[w], gv);
        if constexpr (Q32) atomicAdd(&lds[256 * W + w], hv);
    }
}

// A row's quantized pair as the LDS adds take it: the packed word itself, or (Q32) its g and h apart.
template <bool Q32>
__device__ __forceinline__ void row_units(int32_t word, bool on, int32_t &gv, int32_t &hv) {
    if constexpr (Q32) {
        const int32_t g = packed_g(word);
        gv = on ? g : 0;
        hv = on ? packed_h(word, g) : 0;
    } else {
        gv = on ? word : 0;
        hv = 0;
    }
}

// A dense slab (DP passes): features stacked in the LDS columns by their bin counts, W = 128 columns of 256 bin rows
// and a spare row 256. The feature at row byte i is in column i % 128 at rows [base, base + bins) of it; pos_word[i]
// = base * W + i % 128, and positions past the slab's features point at the spare row (their bytes are 0). A row of
// up to 64 * DP dwords is read by the whole wave, lane l taking dwords l, l + 64, ... (pass p): byte x of dword
// 64p + l is position 256p + 4l + x, so the 32 lanes of a half-wave add to 32 distinct columns, as in a byte slab.
template <int DP>
__device__ __forceinline__ void dense_lanes(const uint32_t *pos_word, uint32_t lane, uint32_t (&xs)[4],
                                            uint32_t (&cols)[DP][4]) {
    const uint32_t rot = (lane & 31u) >> 3;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t x = (k + rot) & 3u;
        xs[k] = 8u * x;
#pragma unroll
        for (int p = 0; p < DP; ++p) cols[p][k] = pos_word[256u * p + 4u * lane + x];
    }
}

// The rows list[c0 .. c1) of a dense slab into the LDS, UNROLL rows a wave at a time over NW waves (`wave` among
// them); dwords past the row (dw_row) read as 0, i.e. bin 0 of spare positions.
template <int W, int DP, int UNROLL, int NW = 16, bool CODES = false>
__device__ __forceinline__ void hist_list_dense(int32_t *lds, const uint32_t *list, uint32_t c0, uint32_t c1,
                                                const int32_t *gh, const uint32_t *bins32, uint32_t dw_row,
                                                const uint32_t (&xs)[4], const uint32_t (&cols)[DP][4],
                                                uint32_t wave = threadIdx.x >> 6, const uint8_t *codes = nullptr) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t last = c1 - 1;
    for (uint32_t base = c0 + wave * UNROLL; base < c1; base += NW * UNROLL) {
        uint32_t r[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) r[u] = list[min(base + u, last)];
        int32_t gq[UNROLL];
        uint32_t dw[UNROLL][DP];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            if constexpr (CODES) gq[u] = code_word(codes[min(base + u, last)]);
            else gq[u] = gh[r[u]];
#pragma unroll
            for (int p = 0; p < DP; ++p) {
                const uint32_t d = 64u * p + lane;
                dw[u][p] = d < dw_row ? bins32[static_cast<size_t>(r[u]) * dw_row + d] : 0u;
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int32_t gv = base + u < c1 ? gq[u] : 0;
#pragma unroll
            for (int p = 0; p < DP; ++p) add_row_bins<W>(lds, dw[u][p], gv, 0, xs, cols[p]);
        }
    }
}

// Loads are branch-free: row positions past the range are clamped to its last row and their gradients
// zeroed, so the compiler issues every load of a step back to back instead of one masked load at a time. A
// wave fetches the row ids of its next step in one coalesced load (lane l: id l) while it works on the current
// step, and hands them out with a shuffle. WIDE: the slab's rows are W / 4 two-byte bins. PACK: the slab's rows
// are W * PACK bytes, PACK features of at most 256 / PACK bins to an LDS column.
template <int W, bool WIDE = false, int PACK = 1, bool Q32 = false, int DP = 0>
__global__ __launch_bounds__(1024) void k_hist(HistArgs a) {
    static_assert(PACK == 1 || (!WIDE && W * PACK <= 256), "a packed row is at most 64 dwords");
    static_assert(!Q32 || W <= 64, "separate g and h counters take twice the LDS");
    static_assert(DP == 0 || (W == 128 && !WIDE && PACK == 1 && !Q32), "a dense slab has 128 byte columns");
    constexpr int DW = WIDE ? W / 8 : W * PACK / 4;  // dwords per row
    constexpr int RPW = WAVE / DW;            // rows per wave step
    // row ids of one step fit one wave-wide load; at W = 128 the 64 accumulator registers leave room for 8
    constexpr int UNROLL = W == 128 ? 8 : (64 / RPW < 16 ? 64 / RPW : 16);
    constexpr uint32_t STEP = 16u * RPW * UNROLL;          // rows per block step (16 waves)
    constexpr int SLOTS = 256 * W / 1024;
    constexpr int LDS_WORDS = (Q32 ? 2 : 1) * 256 * W + (DP ? W : 0);  // a dense slab's spare row
    __shared__ int32_t lds[LDS_WORDS];

    uint32_t lb, n;
    leaf_rows(a.dev_left, a.begin, a.count, a.side, lb, n);
    uint32_t groups, per;
    hist_split(n, a.max_groups, a.min_rows_per_group, groups, per);
    if (blockIdx.x >= groups) return;
    const uint32_t tid = threadIdx.x;
    for (uint32_t k = tid; k < static_cast<uint32_t>(LDS_WORDS); k += 1024) lds[k] = 0;
    int32_t accg[SLOTS], acch[SLOTS];
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) accg[j] = acch[j] = 0;
    __syncthreads();

    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t d = lane % DW, rsub = lane / DW;
    const uint32_t rot = (lane & 31u) >> 3;
    uint32_t xs[4], cols[4];
    row_bin_lanes<W, PACK>(d, rot, xs, cols);
    const uint32_t *rows = a.rows + lb;
    const uint32_t *bins32 = reinterpret_cast<const uint32_t *>(a.bins);
    uint32_t start = blockIdx.x * per;
    uint32_t end = start + per < n ? start + per : n;
    uint32_t dcols[DP ? DP : 1][4];
    if constexpr (DP > 0) dense_lanes<DP>(a.pos_word, lane, xs, dcols);

    for (uint32_t chunk = start; chunk < end; chunk += a.flush_rows) {
        uint32_t cend = end - chunk > a.flush_rows ? chunk + a.flush_rows : end;
        if constexpr (DP > 0) {
            hist_list_dense<W, DP, DP <= 4 ? 4 : 2>(lds, rows, chunk, cend, a.gh, bins32, a.dw_row, xs, dcols);
        } else {
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
                    int32_t gv, hv;
                    row_units<Q32>(g[u], base + u * RPW + rsub < cend, gv, hv);
                    if constexpr (WIDE) add_row_bins_wide<W, Q32>(lds, dw[u], gv, hv, d);
                    else add_row_bins<W, PACK, Q32>(lds, dw[u], gv, hv, xs, cols);
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < SLOTS; ++j) {
            int32_t v = lds[tid + j * 1024];
            lds[tid + j * 1024] = 0;
            if constexpr (Q32) {
                accg[j] += v;
                acch[j] += lds[256 * W + tid + j * 1024];
                lds[256 * W + tid + j * 1024] = 0;
            } else {
                const int32_t gq = packed_g(v);
                accg[j] += gq;
                acch[j] += packed_h(v, gq);
            }
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
    const uint32_t *col_stride;  // flat-histogram bins between a column's consecutive bins: 1, or 4 (wide slab)
    int64_t *out;       // built child's histogram
    int64_t *parent;    // parent's histogram, overwritten with the sibling's (or null)
    const uint32_t *dev_left;
    uint32_t begin, count, side;
    uint32_t max_groups, min_rows_per_group;
    uint32_t width;     // W
    uint32_t seg_shift; // a packed slab's column holds a feature each 2^seg_shift bins: 8 (one feature), 7 or 6
    const uint32_t *slot_flat;  // a dense slab: per slot (bin * W + column) its flat-histogram bin + 1, 0 for none
};

// A block takes 32 slots (bin * W + column) and splits the workgroups' partials of each into 8 stripes that meet in
// LDS. grid: ceil(256 * W / 32) blocks of 256 threads.
__global__ __launch_bounds__(256) void k_hist_reduce(ReduceArgs a) {
    __shared__ int64_t red[2][8][32];
    uint32_t lb, n;
    leaf_rows(a.dev_left, a.begin, a.count, a.side, lb, n);
    uint32_t groups, per;
    hist_split(n, a.max_groups, a.min_rows_per_group, groups, per);
    const uint32_t slots = 256u * a.width;
    const uint32_t tid = threadIdx.x, lane = tid & 31u, stripe = tid >> 5;
    const uint32_t s = blockIdx.x * 32u + lane, col = s % a.width, bin = s / a.width;
    // the slot's feature: segment bin >> seg_shift of the column (its index in the per-feature arrays), its bin;
    // in a dense slab the slot's flat bin from the table
    const uint32_t vb = bin & ((1u << a.seg_shift) - 1u), fs = (bin >> a.seg_shift) * a.width + col;
    const uint32_t flat1 = a.slot_flat && s < slots ? a.slot_flat[s] : 0u;
    const bool on = s < slots && (a.slot_flat ? flat1 != 0u : vb < a.col_bins[fs]);
    int64_t g = 0, h = 0;
    if (on) {
        const int2 *p = reinterpret_cast<const int2 *>(a.partial) + s;
#pragma unroll 8
        for (uint32_t w = stripe; w < groups; w += 8u) {
            const int2 v = p[static_cast<size_t>(w) * slots];
            g += v.x;
            h += v.y;
        }
    }
    red[0][stripe][lane] = g;
    red[1][stripe][lane] = h;
    __syncthreads();
    if (stripe == 0 && on) {
#pragma unroll
        for (int k = 1; k < 8; ++k) {
            g += red[0][k][lane];
            h += red[1][k][lane];
        }
        const size_t o = a.slot_flat ? 2 * static_cast<size_t>(flat1 - 1u)
                                     : 2 * (static_cast<size_t>(a.col_offset[fs]) + static_cast<size_t>(vb) * a.col_stride[fs]);
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
    uint32_t col16, wide;  // u16 column-major bins; the split is a wide feature's numerical rule
    uint32_t *block_left;  // [grid]
    uint32_t *dev_left;    // total left count (written by block 0 of pass 2)
    uint32_t begin, count;
    uint32_t left_bins[8];
    // bagging
    uint32_t bag_seed, bag_round;
    uint64_t row_offset;
    double fraction;
};

// Rows per block for `count` rows over the launch's blocks: a multiple of 256, the same in both passes.
__device__ __forceinline__ uint32_t part_per_block(uint32_t count, uint32_t blocks) {
    uint32_t per = (count + blocks - 1) / blocks;
    per = (per + 1023u) & ~1023u;
    return per < 1024u ? 1024u : per;
}

__device__ __forceinline__ bool part_left(const PartArgs &a, uint32_t row) {
    if (a.col) return rule_left(a.left_bins, a.wide, col_bin(a.col, a.col16, row));
    return static_cast<double>(uniform(a.bag_seed, 2u, a.bag_round, a.row_offset + row)) < a.fraction;
}

// Tiles of 1024 rows: thread t takes rows t, t+256, t+512, t+768 of the tile (four sub-tiles of 256 in order),
// with every load of the tile issued before any is used (positions past the range are clamped and ignored).
__global__ __launch_bounds__(256) void k_part_count(PartArgs a) {
    __shared__ uint32_t wsum[4];
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
    uint32_t wide;     // left_bins hold a numerical rule (rule_left)
};

// `gate` (when set): the leaves of the tree to add, 0 for none (k_tree_nodes).
__global__ void k_add_tree(const uint8_t *__restrict__ colbins, uint32_t col16, uint64_t rows,
                           const DevNode *__restrict__ nodes, const float *__restrict__ leaf_values,
                           float *__restrict__ scores, const uint32_t *gate) {
    if (gate && *gate == 0u) return;
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < rows; r += (uint64_t)gridDim.x * blockDim.x) {
        int32_t node = 0;
        while (node >= 0) {
            const DevNode &nd = nodes[node];
            const uint32_t bin = col_bin(colbins, col16, (size_t)nd.feature * rows + r);
            node = rule_left(nd.left_bins, nd.wide, bin) ? nd.left : nd.right;
        }
        scores[r] += leaf_values[~node];
    }
}

// Each row's leaf from a walk down the tree (nodes in LDS; several rows per thread in flight: the walk is a chain
// of dependent gathers), in row order, and the leaves' exact fixed-point sums rint(v * scale) of the in-bag rows'
// gradients: the sums k_leaf_sums makes over the final partition (integers, so the order does not matter;
// cpu.rs:886-908). grid: any, tl_threads<MAXL>() threads.
struct TreeLeavesArgs {
    const uint8_t *colbins;            // column-major bins [feature][rows]
    uint32_t col16;                    // two bytes per bin
    uint64_t rows;
    const DevNode *nodes;
    uint32_t nn, nl;                   // internal nodes, leaves (nn >= 1, nl <= the kernel's MAXL)
    uint16_t *leaf_of;                 // [rows]
    const float *grad, *hess;          // null: no sums
    float gs, hs;
    unsigned long long *sums;          // [nl][2], zeroed before
    uint32_t bag, bag_seed, bag_round; // bag != 0: only rows in the bag (quantize.rs:147-149) are summed
    uint64_t row_offset;
    double fraction;
    const uint32_t *gate;              // when set: the leaves (nn, nl from it), 0 for no tree (k_tree_nodes)
    const DevScales *dsc;              // when set: gs and hs are its fixed-point scales
};
// Instantiated for trees of up to 512 leaves (28 KiB of LDS: several blocks per compute unit) and up to 2048 (112 KiB:
// one block per compute unit, of 1024 threads, so that 16 waves walk at once). The walk is a chain of dependent
// LDS reads and gathers; its rate is set by the rows in flight, which the register file bounds: 8 rows a thread
// keeps the 512-leaf kernel at 70 registers (7 waves a SIMD), 12 the 2048-leaf one at 124 (4 waves a SIMD, which
// its one block a compute unit fills).
constexpr uint32_t LEAVES_SMALL = 512;
template <uint32_t MAXL> constexpr uint32_t tl_threads() { return MAXL > LEAVES_SMALL ? 1024u : 512u; }
template <uint32_t MAXL> constexpr int tl_rows() { return MAXL > LEAVES_SMALL ? 12 : 8; }

// COL16: two-byte column-major bins (the only kind with numerical rules, `wide`).
template <uint32_t MAXL, bool COL16>
__global__ __launch_bounds__(tl_threads<MAXL>()) void k_tree_leaves(TreeLeavesArgs a) {
    constexpr int RPT = tl_rows<MAXL>();
    constexpr uint32_t NN = MAXL - 1;
    // A level of the walk is branch-free over a thread's RPT rows, so that their LDS reads and gathers issue back to
    // back and each kind waits once: every row reads its node's head (x: its feature's column, bit 31 set for a
    // numerical rule; y: its left and right children as two i16, a leaf l as ~l), gathers its bin, then reads the
    // rule word the bin selects. A row already at its leaf reads node 0 and row 0 and keeps its leaf. The rule words
    // are word-major (word w of node n at w * NN + n).
    __shared__ uint2 head[NN];
    __shared__ uint32_t rule[8 * NN];
    __shared__ unsigned long long ls[MAXL][2];
    uint32_t nn = a.nn, nl = a.nl;
    const float gs = a.dsc ? a.dsc->gsc : a.gs, hs = a.dsc ? a.dsc->hsc : a.hs;
    if (a.gate) {
        nl = *a.gate;
        if (nl == 0u || nl > MAXL) return;
        nn = nl - 1u;
    }
    for (uint32_t k = threadIdx.x; k < nn; k += blockDim.x) {
        const DevNode &x = a.nodes[k];
        head[k] = make_uint2(x.feature | (x.wide ? 0x80000000u : 0u),
                             (static_cast<uint32_t>(x.left) & 0xffffu) | (static_cast<uint32_t>(x.right) << 16));
#pragma unroll
        for (int w = 0; w < 8; ++w) rule[w * NN + k] = x.left_bins[w];
    }
    if (a.grad)
        for (uint32_t l = threadIdx.x; l < nl; l += blockDim.x) ls[l][0] = ls[l][1] = 0ull;
    __syncthreads();
    const uint32_t rows = static_cast<uint32_t>(a.rows);  // rows < 2^32 (row ids are u32)
    const uint32_t step = gridDim.x * blockDim.x;
    for (uint64_t base = blockIdx.x * blockDim.x + threadIdx.x; base < rows; base += static_cast<uint64_t>(RPT) * step) {
        uint32_t r[RPT];
        int32_t nd[RPT];
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
            const uint64_t row = base + static_cast<uint64_t>(k) * step;
            r[k] = row < rows ? static_cast<uint32_t>(row) : 0u;
            nd[k] = row < rows ? 0 : -1;
        }
        for (;;) {
            uint2 h[RPT];
#pragma unroll
            for (int k = 0; k < RPT; ++k) h[k] = head[nd[k] < 0 ? 0 : nd[k]];
            uint32_t b[RPT];
#pragma unroll
            for (int k = 0; k < RPT; ++k) {
                const size_t i = static_cast<size_t>(h[k].x & 0x7fffffffu) * rows + (nd[k] < 0 ? 0u : r[k]);
                b[k] = COL16 ? static_cast<uint32_t>(reinterpret_cast<const uint16_t *>(a.colbins)[i]) : static_cast<uint32_t>(a.colbins[i]);
            }
            uint32_t m0[RPT], m1[RPT];
#pragma unroll
            for (int k = 0; k < RPT; ++k) {
                const uint32_t n = nd[k] < 0 ? 0u : static_cast<uint32_t>(nd[k]);
                const uint32_t w = COL16 ? (h[k].x >> 31 ? 0u : min(b[k] >> 5, 7u)) : b[k] >> 5;
                m0[k] = rule[w * NN + n];
                if (COL16) m1[k] = rule[NN + n];
            }
            bool any = false;
#pragma unroll
            for (int k = 0; k < RPT; ++k) {
                bool left = ((m0[k] >> (b[k] & 31u)) & 1u) != 0u;
                // rule_left's numerical rule: word 0 the threshold, word 1 the NaN bin + 1 or 0
                if (COL16 && (h[k].x >> 31)) left = b[k] <= m0[k] || (m1[k] != 0u && b[k] == m1[k] - 1u);
                const int32_t c = static_cast<int32_t>(static_cast<int16_t>(left ? h[k].y & 0xffffu : h[k].y >> 16));
                nd[k] = nd[k] < 0 ? nd[k] : c;
                any = any || nd[k] >= 0;
            }
            if (!any) break;
        }
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
            if (base + static_cast<uint64_t>(k) * step >= rows) continue;
            const uint32_t leaf = static_cast<uint32_t>(~nd[k]);
            a.leaf_of[r[k]] = static_cast<uint16_t>(leaf);
            if (!a.grad) continue;
            if (a.bag && !(static_cast<double>(uniform(a.bag_seed, 2u, a.bag_round, a.row_offset + r[k])) < a.fraction)) continue;
            atomicAdd(&ls[leaf][0], static_cast<unsigned long long>(to_fixed(a.grad[r[k]], gs)));
            atomicAdd(&ls[leaf][1], static_cast<unsigned long long>(to_fixed(a.hess[r[k]], hs)));
        }
    }
    if (!a.grad) return;
    __syncthreads();
    for (uint32_t l = threadIdx.x; l < nl; l += blockDim.x) {
        if (ls[l][0]) atomicAdd(&a.sums[2 * l], ls[l][0]);
        if (ls[l][1]) atomicAdd(&a.sums[2 * l + 1], ls[l][1]);
    }
}

// scores[r] += the value of row r's leaf: the f32 add of k_add_tree, in row order. Four rows of the grid-stride loop
// at once, their loads (then their leaves' values) issued together: one row an iteration waited on its loads and then
// on its leaf's value (21.0 -> 18.4 us at 10M rows; the gradient kernels, bound by their f64 arithmetic, were slower
// so).
__global__ void k_add_leaf_values(const uint16_t *__restrict__ leaf_of, const float *__restrict__ leaf_values,
                                  float *__restrict__ scores, uint64_t rows, const uint32_t *gate) {
    constexpr int RA = 4;
    if (gate && *gate == 0u) return;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t r0 = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r0 < rows; r0 += RA * stride) {
        uint32_t l[RA];
        float s[RA], v[RA];
#pragma unroll
        for (int k = 0; k < RA; ++k) {
            const uint64_t r = r0 + k * stride;
            l[k] = r < rows ? leaf_of[r] : 0u;
            s[k] = r < rows ? scores[r] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < RA; ++k) v[k] = r0 + k * stride < rows ? leaf_values[l[k]] : 0.0f;
#pragma unroll
        for (int k = 0; k < RA; ++k) {
            const uint64_t r = r0 + k * stride;
            if (r < rows) scores[r] = s[k] + v[k];
        }
    }
}

// a -= b over n int64 values (a histogram slot minus another, learner.rs:365-367)
__global__ void k_sub_i64(int64_t *__restrict__ a, const int64_t *__restrict__ b, uint64_t n) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        a[i] -= b[i];
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
    uint64_t max_cat_to_onehot, max_cat_threshold;
    double cat_l2, cat_smooth;
    int64_t min_data_per_group;
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

// The renewed leaf values of a grown tree from its leaves' fixed-point sums (learner.rs:376-404), shrunk by the
// learning rate (tree.rs:180-185) and, for the first tree, moved by the initial score (tree.rs:188-193, with the
// f32 values added to the scores taken without it: replay.rs:38-40): the host's double operations, in its order.
// One block; leaf l: value[l], weight[l] (double) and lv[l] (the f32 added to the scores).
struct LeafValueArgs {
    const unsigned long long *sums;  // [nl][2] i64 fixed-point {g, h}
    const uint32_t *gate;            // when set: nl from it, 0 for no tree (k_tree_nodes)
    const DevScales *dsc;            // when set: gs and hs are its fixed-point scales
    uint32_t nl, add_bias;
    float gs, hs;                    // the fixed-point scales
    double l1, l2, rate, bias;
    double *value, *weight;
    float *lv;
};

__device__ __forceinline__ double round_to_zero_d(double v) { return fabs(v) > static_cast<double>(1e-35f) ? v : 0.0; }

__global__ void k_leaf_values(LeafValueArgs a) {
    const uint32_t nl = a.gate ? *a.gate : a.nl;
    const float gs = a.dsc ? a.dsc->gsc : a.gs, hs = a.dsc ? a.dsc->hsc : a.hs;
    for (uint32_t l = threadIdx.x; l < nl; l += blockDim.x) {
        const double sg = static_cast<double>(static_cast<int64_t>(a.sums[2 * l])) / static_cast<double>(gs);
        const double sh = static_cast<double>(static_cast<int64_t>(a.sums[2 * l + 1])) / static_cast<double>(hs);
        double v = round_to_zero_d(leaf_output(sg, sh, a.l1, a.l2));
        v = round_to_zero_d(v * a.rate);
        float f = static_cast<float>(v);
        if (a.add_bias) {
            v = round_to_zero_d(v + a.bias);
            f = static_cast<float>(v - a.bias);
        }
        a.value[l] = v;
        a.weight[l] = sh;
        a.lv[l] = f;
    }
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
    uint32_t col;         // the feature's column-major index (its bins for the partition)
    uint32_t nan_idx;     // its NaN bin, or NO_BIN
    uint32_t rule;        // RULE_NUMERICAL, RULE_ONEHOT or RULE_SORTED
    uint32_t cat_forward; // sorted categorical: the run went from the low end of the sorted order
    uint32_t cat_count;   // categorical: bins going left
    uint32_t cat_mask[8]; // categorical: the bins going left
};

constexpr uint32_t NO_BIN = 0xffffffffu;
constexpr uint32_t RULE_NUMERICAL = 0, RULE_ONEHOT = 1, RULE_SORTED = 2;  // split.rs:112-117, 694-844

struct Grown {
    uint32_t bin;
    double ug, uh;
    int64_t count;
    double gain;
};

// Wave-wide inclusive scans with DPP row operations (gfx9: row_shr within rows of 16 lanes, then row_bcast:15
// and row_bcast:31 across rows): each step is a VALU move, not an LDS permute.
constexpr int DPP_ROW_SHR1 = 0x111, DPP_ROW_SHR2 = 0x112, DPP_ROW_SHR4 = 0x114, DPP_ROW_SHR8 = 0x118;
constexpr int DPP_ROW_BCAST15 = 0x142, DPP_ROW_BCAST31 = 0x143;

// The value of the lane the DPP step reads (0 where the step has no source or leaves the lane unwritten).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xf, true));
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    uint32_t lo = dpp_u32<CTRL, ROW_MASK>(static_cast<uint32_t>(v));
    uint32_t hi = dpp_u32<CTRL, ROW_MASK>(static_cast<uint32_t>(v >> 32));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint64_t bits_of(double x) { return __builtin_bit_cast(uint64_t, x); }
__device__ __forceinline__ double double_of(uint64_t x) { return __builtin_bit_cast(double, x); }

// Whether step CTRL/ROW_MASK gives `lane` a source lane (the steps of an inclusive scan, in order).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ bool dpp_has_source(uint32_t lane) {
    const uint32_t row = lane >> 4, in_row = lane & 15u;
    if (CTRL >= DPP_ROW_SHR1 && CTRL <= DPP_ROW_SHR1 + 14) return in_row >= static_cast<uint32_t>(CTRL - 0x110);
    return (ROW_MASK >> row) & 1u;
}

// Inclusive sums over the wave of three exact (integer-valued) quantities.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void scan_add_step(double &g, double &h, int64_t &c) {
    g += double_of(dpp_u64<CTRL, ROW_MASK>(bits_of(g)));
    h += double_of(dpp_u64<CTRL, ROW_MASK>(bits_of(h)));
    c += static_cast<int64_t>(dpp_u64<CTRL, ROW_MASK>(static_cast<uint64_t>(c)));
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, uint32_t lane) {
    uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), lane));
    uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), lane));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// (gain, feature) order of split.rs:866-880 for reductions: a beats b on higher gain, then lower feature; -1 is
// "no candidate".
__device__ __forceinline__ bool cand_better(double ga, int fa, double gb, int fb) {
    return fa >= 0 && (fb < 0 || ga > gb || (ga == gb && fa < fb));
}

// Wave-wide all-reductions through the DPP scan steps; every lane ends with the result.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void best_step(double &g, int &i, uint32_t lane) {
    double og = double_of(dpp_u64<CTRL, ROW_MASK>(bits_of(g)));
    int oi = static_cast<int>(dpp_u32<CTRL, ROW_MASK>(static_cast<uint32_t>(i)));
    if (dpp_has_source<CTRL, ROW_MASK>(lane) && cand_better(og, oi, g, i)) {
        g = og;
        i = oi;
    }
}
// The best (gain, index) pair: higher gain, then the lower index; index < 0 is "none".
__device__ __forceinline__ void wave_best(double &g, int &i) {
    const uint32_t lane = threadIdx.x & 63u;
    best_step<DPP_ROW_SHR1, 0xf>(g, i, lane);
    best_step<DPP_ROW_SHR2, 0xf>(g, i, lane);
    best_step<DPP_ROW_SHR4, 0xf>(g, i, lane);
    best_step<DPP_ROW_SHR8, 0xf>(g, i, lane);
    best_step<DPP_ROW_BCAST15, 0xa>(g, i, lane);
    best_step<DPP_ROW_BCAST31, 0xc>(g, i, lane);
    i = __builtin_amdgcn_readlane(i, 63);
    g = double_of(readlane_u64(bits_of(g), 63));
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void min_step(int &v, uint32_t lane) {
    int o = static_cast<int>(dpp_u32<CTRL, ROW_MASK>(static_cast<uint32_t>(v)));
    if (dpp_has_source<CTRL, ROW_MASK>(lane) && o < v) v = o;
}
__device__ __forceinline__ int wave_min(int v) {
    const uint32_t lane = threadIdx.x & 63u;
    min_step<DPP_ROW_SHR1, 0xf>(v, lane);
    min_step<DPP_ROW_SHR2, 0xf>(v, lane);
    min_step<DPP_ROW_SHR4, 0xf>(v, lane);
    min_step<DPP_ROW_SHR8, 0xf>(v, lane);
    min_step<DPP_ROW_BCAST15, 0xa>(v, lane);
    min_step<DPP_ROW_BCAST31, 0xc>(v, lane);
    return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ double readlane_f64(double v, uint32_t lane) { return double_of(readlane_u64(bits_of(v), lane)); }

// Branch-free all-reductions: a lane without a source in a DPP step reads the reduction's identity (the `old`
// operand with bound_ctrl off), so every step is one move and one max or min.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_min_step(int v) {
    const int o = __builtin_amdgcn_update_dpp(0x7fffffff, v, CTRL, ROW_MASK, 0xf, false);
    return o < v ? o : v;
}
__device__ __forceinline__ int wave_min_i32(int v) {
    v = dpp_min_step<DPP_ROW_SHR1, 0xf>(v);
    v = dpp_min_step<DPP_ROW_SHR2, 0xf>(v);
    v = dpp_min_step<DPP_ROW_SHR4, 0xf>(v);
    v = dpp_min_step<DPP_ROW_SHR8, 0xf>(v);
    v = dpp_min_step<DPP_ROW_BCAST15, 0xa>(v);
    v = dpp_min_step<DPP_ROW_BCAST31, 0xc>(v);
    return __builtin_amdgcn_readlane(v, 63);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_max_step(double v) {  // v is never NaN
    const uint64_t b = bits_of(v), id = bits_of(-__builtin_inf());
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(static_cast<uint32_t>(id)),
                                                                          static_cast<int>(static_cast<uint32_t>(b)), CTRL, ROW_MASK, 0xf, false));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(static_cast<uint32_t>(id >> 32)),
                                                                          static_cast<int>(static_cast<uint32_t>(b >> 32)), CTRL, ROW_MASK, 0xf, false));
    const double o = double_of((static_cast<uint64_t>(hi) << 32) | lo);
    return o > v ? o : v;
}
__device__ __forceinline__ double wave_max_f64(double v) {
    v = dpp_max_step<DPP_ROW_SHR1, 0xf>(v);
    v = dpp_max_step<DPP_ROW_SHR2, 0xf>(v);
    v = dpp_max_step<DPP_ROW_SHR4, 0xf>(v);
    v = dpp_max_step<DPP_ROW_SHR8, 0xf>(v);
    v = dpp_max_step<DPP_ROW_BCAST15, 0xa>(v);
    v = dpp_max_step<DPP_ROW_BCAST31, 0xc>(v);
    return readlane_f64(v, 63);
}
// wave_best for gains that are never NaN: the highest gain, then the lowest index among the lanes holding it.
__device__ __forceinline__ void wave_argmax(double &g, int &i) {
    const double m = wave_max_f64(i >= 0 ? g : -__builtin_inf());
    const int w = wave_min_i32(i >= 0 && g == m ? i : 0x7fffffff);
    g = m;
    i = w == 0x7fffffff ? -1 : w;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_max_u32_step(uint32_t v) {
    const uint32_t o = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xf, false));
    return o > v ? o : v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = dpp_max_u32_step<DPP_ROW_SHR1, 0xf>(v);
    v = dpp_max_u32_step<DPP_ROW_SHR2, 0xf>(v);
    v = dpp_max_u32_step<DPP_ROW_SHR4, 0xf>(v);
    v = dpp_max_u32_step<DPP_ROW_SHR8, 0xf>(v);
    v = dpp_max_u32_step<DPP_ROW_BCAST15, 0xa>(v);
    v = dpp_max_u32_step<DPP_ROW_BCAST31, 0xc>(v);
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_max_u64_step(uint64_t v) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v)), CTRL, ROW_MASK, 0xf, false));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v >> 32)), CTRL, ROW_MASK, 0xf, false));
    const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
    return o > v ? o : v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = dpp_max_u64_step<DPP_ROW_SHR1, 0xf>(v);
    v = dpp_max_u64_step<DPP_ROW_SHR2, 0xf>(v);
    v = dpp_max_u64_step<DPP_ROW_SHR4, 0xf>(v);
    v = dpp_max_u64_step<DPP_ROW_SHR8, 0xf>(v);
    v = dpp_max_u64_step<DPP_ROW_BCAST15, 0xa>(v);
    v = dpp_max_u64_step<DPP_ROW_BCAST31, 0xc>(v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), 63));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), 63));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
// wave_max_u64 by the high words first: their u32 maximum, then the low word of the one lane holding it, or the low
// words' maximum over the lanes holding it when several do (half the DPP work of wave_max_u64 when the high words
// rarely tie). All lanes active.
__device__ __forceinline__ uint64_t wave_max_u64_hi(uint64_t v) {
    const uint32_t hi = static_cast<uint32_t>(v >> 32), lo = static_cast<uint32_t>(v);
    const uint32_t mh = wave_max_u32(hi);
    const unsigned long long at = __ballot(hi == mh);
    const uint32_t ml = (at & (at - 1ull)) == 0ull
                            ? static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lo), static_cast<int>(__builtin_ctzll(at))))
                            : wave_max_u32(hi == mh ? lo : 0u);
    return (static_cast<uint64_t>(mh) << 32) | ml;
}

// A feature candidate as held by lane `owner`, broadcast to the wave.
__device__ __forceinline__ FeatCand readlane_cand(const FeatCand &c, uint32_t owner) {
    FeatCand r;
    r.found = __builtin_amdgcn_readlane(c.found, owner);
    r.splittable = __builtin_amdgcn_readlane(c.splittable, owner);
    r.gain = readlane_f64(c.gain, owner);
    r.best_gain = readlane_f64(c.best_gain, owner);
    r.threshold = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(c.threshold), owner));
    r.default_left = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(c.default_left), owner));
    r.left_grad = readlane_f64(c.left_grad, owner);
    r.left_hess = readlane_f64(c.left_hess, owner);
    r.left_count = static_cast<int64_t>(readlane_u64(static_cast<uint64_t>(c.left_count), owner));
    r.left_units_g = readlane_f64(c.left_units_g, owner);
    r.left_units_h = readlane_f64(c.left_units_h, owner);
    r.col = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(c.col), owner));
    r.nan_idx = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(c.nan_idx), owner));
    r.rule = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(c.rule), owner));
    r.cat_forward = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(c.cat_forward), owner));
    r.cat_count = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(c.cat_count), owner));
#pragma unroll
    for (int w = 0; w < 8; ++w)
        r.cat_mask[w] = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(c.cat_mask[w]), owner));
    return r;
}


struct FeatDev {
    uint32_t num_bins, hist_offset, kind, nan_bin;
    uint32_t col;   // column-major index among the non-trivial features
    uint32_t wide;  // two-byte bins (up to 1024, numerical): splits carry a numerical rule (rule_left)
};

struct ScanJob {
    const int64_t *hist;  // the leaf's histogram
    double units_grad, units_hess;
    int64_t count;
    FeatCand *out;        // [num_features]
};

// split.rs:584-620 find_numerical: the reverse scan (split.rs:557-567: missing values go left) always; the forward
// scan over the bins before the NaN bin (split.rs:571-580) only for a feature with a NaN bin and more than two bins.
__device__ __forceinline__ bool scan_searched(const Ctx &c, const FeatDev &m, bool evaluate) {
    return c.valid && evaluate && m.num_bins >= 2 && (m.kind == 1 || m.kind == 2);
}
__device__ __forceinline__ bool scan_two_way(const FeatDev &m) { return m.nan_bin && m.num_bins > 2; }

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_max_i32_step(int v) {
    const int o = __builtin_amdgcn_update_dpp(static_cast<int>(0x80000000u), v, CTRL, ROW_MASK, 0xf, false);
    return o > v ? o : v;
}
__device__ __forceinline__ int wave_max_i32(int v) {
    v = dpp_max_i32_step<DPP_ROW_SHR1, 0xf>(v);
    v = dpp_max_i32_step<DPP_ROW_SHR2, 0xf>(v);
    v = dpp_max_i32_step<DPP_ROW_SHR4, 0xf>(v);
    v = dpp_max_i32_step<DPP_ROW_SHR8, 0xf>(v);
    v = dpp_max_i32_step<DPP_ROW_BCAST15, 0xa>(v);
    v = dpp_max_i32_step<DPP_ROW_BCAST31, 0xc>(v);
    return __builtin_amdgcn_readlane(v, 63);
}

// One candidate of a scan (split.rs:420-462): the accumulated side's exact units and rows; returns its gain, -inf
// when the candidate is skipped (that side too small) or NaN (split.rs:508-531), and sets `stop` when the other side
// is too small while this one is not (the reference's `break`).
__device__ __forceinline__ double candidate_gain(const Ctx &c, const SplitCfgDev &cfg, double ug, double uh, int64_t cnt,
                                                int64_t min_count, bool &stop) {
    const double hh = K_EPSILON + uh * c.scale_hess;
    const bool skip = cnt < min_count || hh < cfg.min_sum_hessian_in_leaf || uh <= 0.0;
    const bool other_small = c.num_data - cnt < min_count || c.sum_hess - hh < cfg.min_sum_hessian_in_leaf ||
                             c.units_hess - uh <= 0.0;
    stop = other_small && !skip;
    const double gg = ug * c.scale_grad;
    const double gain = leaf_gain(c.sum_grad - gg, c.sum_hess - hh, cfg.lambda_l1, cfg.lambda_l2) +
                        leaf_gain(gg, hh, cfg.lambda_l1, cfg.lambda_l2);
    return (skip || gain != gain) ? -__builtin_inf() : gain;
}

// A candidate's stop test alone (candidate_gain's `stop`, without the gain).
__device__ __forceinline__ bool candidate_stop(const Ctx &c, const SplitCfgDev &cfg, double uh, int64_t cnt,
                                               int64_t min_count) {
    const double hh = K_EPSILON + uh * c.scale_hess;
    const bool skip = cnt < min_count || hh < cfg.min_sum_hessian_in_leaf || uh <= 0.0;
    const bool other_small = c.num_data - cnt < min_count || c.sum_hess - hh < cfg.min_sum_hessian_in_leaf ||
                             c.units_hess - uh <= 0.0;
    return other_small && !skip;
}

constexpr uint32_t UNIT_FEATS = 16;  // features a scan unit holds at most (segments of 4 lanes)

// A scan's lanes: the wave (SEGL = 64), or segments of SEGL = 16 or 4 lanes, each scanning its own feature of at most
// 4 * SEGL bins (t = lane % SEGL holds bins 4t .. 4t + 3). The wave-wide operations below, taken over a segment:
// inclusive sums (DPP row shifts stay inside a row of 16 lanes; a 4-lane segment masks the lanes below the shift),
// the segment's last value, maxima and minima, and a lane's value read by its segment.
template <int SEGL>
__device__ __forceinline__ void seg_scan_add(double &g, double &h, int64_t &c) {
    if constexpr (SEGL == 64) {
        scan_add_step<DPP_ROW_SHR1, 0xf>(g, h, c);
        scan_add_step<DPP_ROW_SHR2, 0xf>(g, h, c);
        scan_add_step<DPP_ROW_SHR4, 0xf>(g, h, c);
        scan_add_step<DPP_ROW_SHR8, 0xf>(g, h, c);
        scan_add_step<DPP_ROW_BCAST15, 0xa>(g, h, c);
        scan_add_step<DPP_ROW_BCAST31, 0xc>(g, h, c);
    } else if constexpr (SEGL == 16) {
        scan_add_step<DPP_ROW_SHR1, 0xf>(g, h, c);
        scan_add_step<DPP_ROW_SHR2, 0xf>(g, h, c);
        scan_add_step<DPP_ROW_SHR4, 0xf>(g, h, c);
        scan_add_step<DPP_ROW_SHR8, 0xf>(g, h, c);
    } else {
        static_assert(SEGL == 4, "segments of 64, 16 or 4 lanes");
        const uint32_t t = threadIdx.x & 3u;
        const double g1 = double_of(dpp_u64<DPP_ROW_SHR1, 0xf>(bits_of(g))), h1 = double_of(dpp_u64<DPP_ROW_SHR1, 0xf>(bits_of(h)));
        const int64_t c1 = static_cast<int64_t>(dpp_u64<DPP_ROW_SHR1, 0xf>(static_cast<uint64_t>(c)));
        if (t >= 1) {
            g += g1;
            h += h1;
            c += c1;
        }
        const double g2 = double_of(dpp_u64<DPP_ROW_SHR2, 0xf>(bits_of(g))), h2 = double_of(dpp_u64<DPP_ROW_SHR2, 0xf>(bits_of(h)));
        const int64_t c2 = static_cast<int64_t>(dpp_u64<DPP_ROW_SHR2, 0xf>(static_cast<uint64_t>(c)));
        if (t >= 2) {
            g += g2;
            h += h2;
            c += c2;
        }
    }
}
template <int SEGL>
__device__ __forceinline__ double seg_read_f64(double v, uint32_t t) {
    if constexpr (SEGL == 64) return readlane_f64(v, t);
    else return __shfl(v, static_cast<int>(t), SEGL);
}
template <int SEGL>
__device__ __forceinline__ int64_t seg_read_i64(int64_t v, uint32_t t) {
    if constexpr (SEGL == 64) return static_cast<int64_t>(readlane_u64(static_cast<uint64_t>(v), t));
    else return static_cast<int64_t>(__shfl(static_cast<long long>(v), static_cast<int>(t), SEGL));
}
template <int SEGL>
__device__ __forceinline__ int seg_max_i32(int v) {
    if constexpr (SEGL == 64) {
        return wave_max_i32(v);
    } else {
#pragma unroll
        for (int o = SEGL / 2; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, SEGL));
        return v;
    }
}
template <int SEGL>
__device__ __forceinline__ int seg_min_i32(int v) {
    if constexpr (SEGL == 64) {
        return wave_min_i32(v);
    } else {
#pragma unroll
        for (int o = SEGL / 2; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, SEGL));
        return v;
    }
}
template <int SEGL>
__device__ __forceinline__ double seg_max_f64(double v) {  // v is never NaN
    if constexpr (SEGL == 64) {
        return wave_max_f64(v);
    } else {
#pragma unroll
        for (int o = SEGL / 2; o > 0; o >>= 1) {
            const double w = __shfl_xor(v, o, SEGL);
            v = w > v ? w : v;
        }
        return v;
    }
}

// scan_numerical for a feature of up to 1024 bins (two-byte bins, an extension): lane l holds bins
// 16l .. 16l + 15. The same candidates, stops and ties as scan_numerical, in two passes over the lane's bins so that
// only the units stay in registers: the first finds both directions' stops, the second evaluates the candidates in
// range, re-forming the exact prefix sums as it goes.
__device__ void scan_numerical_wide(const Ctx &c, const SplitCfgDev &cfg, const FeatDev &m, const int64_t *hist,
                                    bool &rf, Grown &rg, bool &ff, Grown &fg) {
    constexpr int NPB = 16;
    const int lane = static_cast<int>(threadIdx.x & 63u);
    const int64_t *h = hist + 2 * static_cast<size_t>(m.hist_offset);
    const int nb = static_cast<int>(m.num_bins);
    const bool two = scan_two_way(m);
    const int top = two ? nb - 2 : nb - 1;
    double gu[NPB], hu[NPB];
#pragma unroll
    for (int j = 0; j < NPB; ++j) {
        const int b = NPB * lane + j;
        const int t = b <= top ? b : 0;
        gu[j] = b <= top ? static_cast<double>(h[2 * t]) : 0.0;
        hu[j] = b <= top ? static_cast<double>(h[2 * t + 1]) : 0.0;
    }
    // per-bin counts (split.rs:196-198): `(x + 0.5) as i64`
    auto count_of = [&](int j) {
        return NPB * lane + j <= top ? sat_i64(hu[j] * c.scale_hess * c.cnt_factor + 0.5) : int64_t{0};
    };
    double lg = 0.0, lh = 0.0;
    int64_t lc = 0;
#pragma unroll
    for (int j = 0; j < NPB; ++j) {
        lg += gu[j];
        lh += hu[j];
        lc += count_of(j);
    }
    double eg = lg, eh = lh;
    int64_t ec = lc;
    scan_add_step<DPP_ROW_SHR1, 0xf>(eg, eh, ec);
    scan_add_step<DPP_ROW_SHR2, 0xf>(eg, eh, ec);
    scan_add_step<DPP_ROW_SHR4, 0xf>(eg, eh, ec);
    scan_add_step<DPP_ROW_SHR8, 0xf>(eg, eh, ec);
    scan_add_step<DPP_ROW_BCAST15, 0xa>(eg, eh, ec);
    scan_add_step<DPP_ROW_BCAST31, 0xc>(eg, eh, ec);
    const double tg = readlane_f64(eg, 63), th = readlane_f64(eh, 63);
    const int64_t tc = static_cast<int64_t>(readlane_u64(static_cast<uint64_t>(ec), 63));
    eg -= lg;
    eh -= lh;
    ec -= lc;
    const int64_t min_count = cfg.min_data_in_leaf > 1 ? cfg.min_data_in_leaf : 1;
    // pass 1: the stops (reverse: the highest stopping bin; forward: the lowest)
    int stop_r = -1, stop_f = 0x7fffffff;
    {
        double pg = eg, ph = eh;
        int64_t pc = ec;
        for (int j = 0; j < NPB; ++j) {
            const int b = NPB * lane + j;
            const int64_t cj = count_of(j);
            const double bg = pg, bh = ph;  // the prefix below b
            const int64_t bc = pc;
            pg += gu[j];
            ph += hu[j];
            pc += cj;
            if (b > top) continue;
            if (b >= 1 && candidate_stop(c, cfg, th - bh, tc - bc, min_count)) stop_r = b;
            if (two && stop_f == 0x7fffffff && candidate_stop(c, cfg, ph, pc, min_count)) stop_f = b;
            (void)bg;
        }
    }
    const int lo = wave_max_i32(stop_r) + 1;
    const int hi = two ? wave_min_i32(stop_f) : 0;
    // pass 2: the candidates in range; each lane keeps its best of each direction with its accumulated side
    double brg = -__builtin_inf(), bfg = -__builtin_inf();
    int brb = -1, bfb = -1;
    double rug = 0.0, ruh = 0.0, fug = 0.0, fuh = 0.0;
    int64_t ruc = 0, fuc = 0;
    {
        double pg = eg, ph = eh;
        int64_t pc = ec;
        for (int j = 0; j < NPB; ++j) {
            const int b = NPB * lane + j;
            const int64_t cj = count_of(j);
            const double ag = tg - pg, ah = th - ph;  // the right side from b up
            const int64_t ac = tc - pc;
            pg += gu[j];
            ph += hu[j];
            pc += cj;
            if (b > top) continue;
            bool stop;
            if (b >= 1 && b >= lo) {
                const double gv = candidate_gain(c, cfg, ag, ah, ac, min_count, stop);
                if (brb < 0 || gv >= brg) {  // visited downward: the highest b on equal gains
                    brg = gv;
                    brb = b;
                    rug = ag;
                    ruh = ah;
                    ruc = ac;
                }
            }
            if (two && b < hi) {
                const double gv = candidate_gain(c, cfg, pg, ph, pc, min_count, stop);
                if (bfb < 0 || gv > bfg) {  // visited upward: the lowest b on equal gains
                    bfg = gv;
                    bfb = b;
                    fug = pg;
                    fuh = ph;
                    fuc = pc;
                }
            }
        }
    }
    rf = false;
    ff = false;
    {
        const double best = wave_max_f64(brb >= 0 ? brg : -__builtin_inf());
        const int first = wave_max_i32(brb >= 0 && brg == best ? brb : -1);
        if (first >= 0 && best > c.min_gain_shift) {
            const uint32_t owner = static_cast<uint32_t>(first) / NPB;
            rg.ug = readlane_f64(rug, owner);
            rg.uh = readlane_f64(ruh, owner);
            rg.count = static_cast<int64_t>(readlane_u64(static_cast<uint64_t>(ruc), owner));
            rg.gain = best;
            rg.bin = static_cast<uint32_t>(first);
            rf = true;
        }
    }
    if (two) {
        const double best = wave_max_f64(bfb >= 0 ? bfg : -__builtin_inf());
        const int first = wave_min_i32(bfb >= 0 && bfg == best ? bfb : 0x7fffffff);
        if (first != 0x7fffffff && best > c.min_gain_shift) {
            const uint32_t owner = static_cast<uint32_t>(first) / NPB;
            fg.ug = readlane_f64(fug, owner);
            fg.uh = readlane_f64(fuh, owner);
            fg.count = static_cast<int64_t>(readlane_u64(static_cast<uint64_t>(fuc), owner));
            fg.gain = best;
            fg.bin = static_cast<uint32_t>(first);
            ff = true;
        }
    }
}

// Both scan directions of a numerical feature (split.rs:555-620) from one pass over its bins, wave-wide. Lane l
// holds bins 4l .. 4l + 3 in natural order; the scanned bins are 0 .. top, top being the last bin before the NaN bin
// when the feature scans both ways and the last bin otherwise. Every accumulated side is a sum of exact integers
// (histogram units, per-bin counts rounded as split.rs:196-198), so the reverse scan's right side from bin b up is
// the total minus the prefix below b, the same values the reference's running sums reach.
// - Reverse (missing values go left): visits b = top .. 1; stops at the first b, in that order the highest, where
//   the other side is too small while the accumulated one is not; keeps the first maximum in its order, so the
//   highest b on equal gains. Threshold b - 1.
// - Forward (missing values go right; two-way features only): visits b = 0 .. top; stops at the lowest such b;
//   keeps the lowest b on equal gains. Threshold b.
template <int SEGL = 64>
__device__ void scan_numerical(const Ctx &c, const SplitCfgDev &cfg, const FeatDev &m, const int64_t *hist, bool &rf,
                               Grown &rg, bool &ff, Grown &fg) {
    const int lane = static_cast<int>(threadIdx.x & static_cast<uint32_t>(SEGL - 1));  // the lane in its segment
    const int64_t *h = hist + 2 * static_cast<size_t>(m.hist_offset);
    const int nb = static_cast<int>(m.num_bins);
    const bool two = scan_two_way(m);
    const int top = two ? nb - 2 : nb - 1;
    double gu[4], hu[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = 4 * lane + j;
        const int t = b <= top ? b : 0;
        gu[j] = b <= top ? static_cast<double>(h[2 * t]) : 0.0;
        hu[j] = b <= top ? static_cast<double>(h[2 * t + 1]) : 0.0;
    }
    // per-bin counts: `(x + 0.5) as i64`, one conversion when the wave's are all in u32
    double xc[4];
    bool small = true;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        xc[j] = 4 * lane + j <= top ? hu[j] * c.scale_hess * c.cnt_factor + 0.5 : 0.0;
        small = small && xc[j] >= 0.0 && xc[j] < 4294967296.0;
    }
    int64_t ci[4];
    if (__all(small)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) ci[j] = static_cast<int64_t>(static_cast<uint32_t>(xc[j]));
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) ci[j] = sat_i64(xc[j]);
    }
    // inclusive prefix P(b) over bins 0 .. top
    double pg[4], ph[4];
    int64_t pc[4];
    double lg = 0.0, lh = 0.0;
    int64_t lc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        lg += gu[j];
        lh += hu[j];
        lc += ci[j];
        pg[j] = lg;
        ph[j] = lh;
        pc[j] = lc;
    }
    double eg = lg, eh = lh;
    int64_t ec = lc;
    seg_scan_add<SEGL>(eg, eh, ec);
    const double tg = seg_read_f64<SEGL>(eg, SEGL - 1), th = seg_read_f64<SEGL>(eh, SEGL - 1);
    const int64_t tc = seg_read_i64<SEGL>(ec, SEGL - 1);
    eg -= lg;
    eh -= lh;
    ec -= lc;
    const int64_t min_count = cfg.min_data_in_leaf > 1 ? cfg.min_data_in_leaf : 1;
    double rgu[4], rhu[4], grv[4], gfv[4];
    int64_t rcu[4];
    int stop_r = -1, stop_f = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = 4 * lane + j;
        pg[j] += eg;
        ph[j] += eh;
        pc[j] += ec;
        // reverse: the right side from bin b up
        rgu[j] = tg - (pg[j] - gu[j]);
        rhu[j] = th - (ph[j] - hu[j]);
        rcu[j] = tc - (pc[j] - ci[j]);
        grv[j] = -__builtin_inf();
        gfv[j] = -__builtin_inf();
        if (b <= top) {
            bool stop = false;
            if (b >= 1) {
                grv[j] = candidate_gain(c, cfg, rgu[j], rhu[j], rcu[j], min_count, stop);
                if (stop) stop_r = b;  // b grows with j: the lane's highest
            }
            if (two) {
                gfv[j] = candidate_gain(c, cfg, pg[j], ph[j], pc[j], min_count, stop);
                if (stop && stop_f == 0x7fffffff) stop_f = b;  // the lane's lowest
            }
        }
    }
    rf = false;
    ff = false;
    {  // reverse: candidates above the highest stop, the highest b among equal gains
        const int lo = seg_max_i32<SEGL>(stop_r) + 1;  // >= 0
        double bg = -__builtin_inf();
        int bb = -1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int b = 4 * lane + j;
            if (b >= 1 && b >= lo && b <= top && (bb < 0 || grv[j] >= bg)) {
                bg = grv[j];
                bb = b;
            }
        }
        const double best = seg_max_f64<SEGL>(bb >= 0 ? bg : -__builtin_inf());
        const int first = seg_max_i32<SEGL>(bb >= 0 && bg == best ? bb : -1);
        if (first >= 0 && best > c.min_gain_shift) {
            const uint32_t owner = static_cast<uint32_t>(first) >> 2;
            const int jj = first & 3;
            double og = 0.0, oh = 0.0;
            int64_t oc = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (j == jj) {
                    og = rgu[j];
                    oh = rhu[j];
                    oc = rcu[j];
                }
            rg.ug = seg_read_f64<SEGL>(og, owner);
            rg.uh = seg_read_f64<SEGL>(oh, owner);
            rg.count = seg_read_i64<SEGL>(oc, owner);
            rg.gain = best;
            rg.bin = static_cast<uint32_t>(first);
            rf = true;
        }
    }
    if (two) {  // forward: candidates below the lowest stop, the lowest b among equal gains
        const int hi = seg_min_i32<SEGL>(stop_f);
        double bg = -__builtin_inf();
        int bb = -1;
#pragma unroll
        for (int j = 3; j >= 0; --j) {
            const int b = 4 * lane + j;
            if (b < hi && b <= top && (bb < 0 || gfv[j] >= bg)) {
                bg = gfv[j];
                bb = b;
            }
        }
        const double best = seg_max_f64<SEGL>(bb >= 0 ? bg : -__builtin_inf());
        const int first = seg_min_i32<SEGL>(bb >= 0 && bg == best ? bb : 0x7fffffff);
        if (first != 0x7fffffff && best > c.min_gain_shift) {
            const uint32_t owner = static_cast<uint32_t>(first) >> 2;
            const int jj = first & 3;
            double og = 0.0, oh = 0.0;
            int64_t oc = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (j == jj) {
                    og = pg[j];
                    oh = ph[j];
                    oc = pc[j];
                }
            fg.ug = seg_read_f64<SEGL>(og, owner);
            fg.uh = seg_read_f64<SEGL>(oh, owner);
            fg.count = seg_read_i64<SEGL>(oc, owner);
            fg.gain = best;
            fg.bin = static_cast<uint32_t>(first);
            ff = true;
        }
    }
}

// The feature's candidate from its scans' results (rf/rg reverse, ff/fg forward).
__device__ FeatCand feature_candidate(const Ctx &c, const FeatDev &m, bool rf, const Grown &rg, bool ff, const Grown &fg) {
    FeatCand r = {};
    bool have = false;
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
        r.default_left = scan_two_way(m) ? 1 : (m.nan_bin ? 0 : 1);
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
    if (have) {
        r.found = 1;
        r.gain = r.best_gain - c.min_gain_shift;
        r.col = m.col;
        r.nan_idx = m.nan_bin ? m.num_bins - 1 : NO_BIN;
    }
    return r;
}

// ---------------------------------------------------------------------------------------------------------
// Categorical features (split.rs:694-844): one-hot for at most max_cat_to_onehot bins, otherwise the bins with
// enough rows sorted by their smoothed gradient ratio and scanned from both ends. One wave per feature.
// ---------------------------------------------------------------------------------------------------------

// split.rs:243-258 check for a growing side (rows, hessian, hessian units) against the other side:
// 0 skip the candidate (Continue), 1 stop the scan (Break), 2 evaluate it.
__device__ __forceinline__ int side_check(const Ctx &c, const SplitCfgDev &cfg, int64_t cnt, double hess, double units_h,
                                          int64_t other_cnt, double other_hess) {
    if (cnt < cfg.min_data_in_leaf || cnt <= 0 || hess < cfg.min_sum_hessian_in_leaf || units_h <= 0.0) return 0;
    if (other_cnt < cfg.min_data_in_leaf || other_cnt <= 0) return 1;
    if (other_hess < cfg.min_sum_hessian_in_leaf || c.units_hess - units_h <= 0.0) return 1;
    return 2;
}

__device__ __forceinline__ int64_t bin_rows(const Ctx &c, double units_h) {  // split.rs:236-238 bin_count
    return sat_i64(units_h * c.scale_hess * c.cnt_factor + 0.5);
}

__device__ __forceinline__ void mask_set(uint32_t (&mask)[8], uint32_t bin) {
#pragma unroll
    for (uint32_t w = 0; w < 8; ++w)
        if ((bin >> 5) == w) mask[w] |= 1u << (bin & 31u);
}

// split.rs:695-736 find_onehot: every bin 1..num_bins on its own against the rest; the first strict maximum above
// min_gain_shift (NaN never counts). Lane l takes bins 1 + l + 64 j.
__device__ FeatCand onehot_scan(const Ctx &c, const SplitCfgDev &cfg, const FeatDev &m, const int64_t *hist) {
    const int64_t *h = hist + 2 * static_cast<size_t>(m.hist_offset);
    const uint32_t lane = threadIdx.x & 63u;
    const int nb = static_cast<int>(m.num_bins);
    double bg = 0.0, bu_g = 0.0, bu_h = 0.0;
    int bt = -1;
    int64_t bcnt = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = 1 + static_cast<int>(lane) + 64 * j;
        if (t >= nb) continue;
        const double ug = static_cast<double>(h[2 * t]), uh = static_cast<double>(h[2 * t + 1]);
        const int64_t cnt = bin_rows(c, uh);
        const double raw_hess = uh * c.scale_hess;
        const int64_t other_cnt = c.num_data - cnt;
        const double other_hess = c.sum_hess - raw_hess - K_EPSILON;
        if (side_check(c, cfg, cnt, raw_hess, uh, other_cnt, other_hess) != 2) continue;
        const double grad = ug * c.scale_grad;
        const double gain = leaf_gain(c.sum_grad - grad, other_hess, cfg.lambda_l1, cfg.lambda_l2) +
                            leaf_gain(grad, raw_hess + K_EPSILON, cfg.lambda_l1, cfg.lambda_l2);
        if (gain != gain || gain <= c.min_gain_shift) continue;
        if (bt < 0 || gain > bg) {
            bg = gain;
            bt = t;
            bu_g = ug;
            bu_h = uh;
            bcnt = cnt;
        }
    }
    const bool any = __ballot(bt >= 0) != 0;
    double wg = bg;
    int wt = bt;
    wave_best(wg, wt);
    FeatCand r = {};
    r.splittable = any ? 1 : 0;
    if (wt >= 0) {
        const uint32_t owner = static_cast<uint32_t>(wt - 1) & 63u;
        const double ug = readlane_f64(bu_g, owner), uh = readlane_f64(bu_h, owner);
        const int64_t cnt = static_cast<int64_t>(readlane_u64(static_cast<uint64_t>(bcnt), owner));
        r.found = 1;
        r.best_gain = wg;
        r.gain = wg - c.min_gain_shift;
        r.threshold = static_cast<uint32_t>(wt);
        r.left_grad = ug * c.scale_grad;
        r.left_hess = uh * c.scale_hess + K_EPSILON;
        r.left_count = cnt;
        r.left_units_g = ug;
        r.left_units_h = uh;
        r.col = m.col;
        r.nan_idx = NO_BIN;
        r.rule = RULE_ONEHOT;
        r.cat_count = 1;
        mask_set(r.cat_mask, static_cast<uint32_t>(wt));
    }
    return r;
}

// A wave's LDS for the sorted categorical scan.
struct CatScratch {
    unsigned long long key[256];  // total-order bits of each bin's ratio (bin-indexed)
    uint32_t order[256];          // the sorted bins
    uint8_t eligible[256];        // the bin has at least cat_smooth rows
};

// f64 total order (split.rs:754 total_cmp) as an unsigned integer order. A ratio that is NaN (0 / 0 with
// cat_smooth = 0) orders by its sign bit; the reference computes it on x86-64, whose invalid-operation result is the
// default NaN with the sign set, so the device's NaN is replaced by that one.
__device__ __forceinline__ unsigned long long total_order_bits(double x) {
    unsigned long long b = x != x ? 0xfff8000000000000ull : __builtin_bit_cast(unsigned long long, x);
    return (b >> 63) ? ~b : (b | 0x8000000000000000ull);
}

// One run of split.rs:795-843 SortedScan::run over the first `steps` positions of the sorted order, from the low
// end (forward) or the high end. Positions i = lane + 64 j; the stateful min_data_per_group walk is uniform.
// Returns whether a candidate passed; (gain, pos) the best, and its left sums.
__device__ bool sorted_run(const Ctx &c, const SplitCfgDev &cfg, const int64_t *h, const CatScratch &sc, int used,
                           int steps, bool forward, double l2, bool &splittable, double &best_gain, int &best_pos,
                           double &lug, double &luh, int64_t &lcnt) {
    const uint32_t lane = threadIdx.x & 63u;
    double pg[4], ph[4];
    int64_t pc[4], ci[4];
    double lg = 0.0, lh = 0.0;
    int64_t lc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = static_cast<int>(lane) * 4 + j;  // contiguous positions per lane: the prefix below is in order
        double gu = 0.0, hu = 0.0;
        int64_t cn = 0;
        if (i < steps) {
            const uint32_t t = sc.order[forward ? i : used - 1 - i];
            gu = static_cast<double>(h[2 * t]);
            hu = static_cast<double>(h[2 * t + 1]);
            cn = bin_rows(c, hu);
        }
        ci[j] = cn;
        lg += gu;
        lh += hu;
        lc += cn;
        pg[j] = lg;
        ph[j] = lh;
        pc[j] = lc;
    }
    double eg = lg, eh = lh;
    int64_t ec = lc;
    scan_add_step<DPP_ROW_SHR1, 0xf>(eg, eh, ec);
    scan_add_step<DPP_ROW_SHR2, 0xf>(eg, eh, ec);
    scan_add_step<DPP_ROW_SHR4, 0xf>(eg, eh, ec);
    scan_add_step<DPP_ROW_SHR8, 0xf>(eg, eh, ec);
    scan_add_step<DPP_ROW_BCAST15, 0xa>(eg, eh, ec);
    scan_add_step<DPP_ROW_BCAST31, 0xc>(eg, eh, ec);
    eg -= lg;
    eh -= lh;
    ec -= lc;
    // per position: 1 skip (Continue), 2 stop (Break, or the other side below min_data_per_group), 0 candidate
    uint32_t flags = 0;  // 2 bits per position j
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        pg[j] += eg;
        ph[j] += eh;
        pc[j] += ec;
        const int i = static_cast<int>(lane) * 4 + j;
        if (i >= steps) continue;
        const double lhess = K_EPSILON + ph[j] * c.scale_hess;
        const int64_t rcnt = c.num_data - pc[j];
        const double rhess = c.sum_hess - lhess;
        const int chk = side_check(c, cfg, pc[j], lhess, ph[j], rcnt, rhess);
        uint32_t f = chk == 0 ? 1u : (chk == 1 || rcnt < cfg.min_data_per_group ? 2u : 0u);
        flags |= f << (2 * j);
    }
    // the walk (split.rs:806-823): rows since the last evaluated candidate must reach min_data_per_group
    uint32_t mine = 0;  // bit j: this lane's position 4 lane + j is evaluated
    int64_t group = 0;
    for (int i = 0; i < steps; ++i) {
        const uint32_t src = static_cast<uint32_t>(i) >> 2, jj = static_cast<uint32_t>(i) & 3u;
        const int64_t cij = jj == 0 ? ci[0] : (jj == 1 ? ci[1] : (jj == 2 ? ci[2] : ci[3]));
        group += static_cast<int64_t>(readlane_u64(static_cast<uint64_t>(cij), src));
        const uint32_t f = (static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(flags), src)) >> (2 * jj)) & 3u;
        if (f == 1u) continue;
        if (f == 2u) break;
        if (group < cfg.min_data_per_group) continue;
        group = 0;
        if (lane == src) mine |= 1u << jj;
    }
    double bg = 0.0;
    int bp = -1;
    double b_g = 0.0, b_h = 0.0;
    int64_t b_c = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (!((mine >> j) & 1u)) continue;
        const double lgrad = pg[j] * c.scale_grad;
        const double lhess = K_EPSILON + ph[j] * c.scale_hess;
        const double rhess = c.sum_hess - lhess;
        const double gain = leaf_gain(lgrad, lhess, cfg.lambda_l1, l2) + leaf_gain(c.sum_grad - lgrad, rhess, cfg.lambda_l1, l2);
        if (gain != gain || gain <= c.min_gain_shift) continue;
        if (bp < 0 || gain > bg) {
            bg = gain;
            bp = static_cast<int>(lane) * 4 + j;
            b_g = pg[j];
            b_h = ph[j];
            b_c = pc[j];
        }
    }
    splittable = splittable || (__ballot(bp >= 0) != 0);
    double wg = bg;
    int wp = bp;
    wave_best(wg, wp);
    if (wp < 0) return false;
    const uint32_t owner = static_cast<uint32_t>(wp) >> 2;
    best_gain = wg;
    best_pos = wp;
    lug = readlane_f64(b_g, owner);
    luh = readlane_f64(b_h, owner);
    lcnt = static_cast<int64_t>(readlane_u64(static_cast<uint64_t>(b_c), owner));
    return true;
}

// split.rs:740-784: sorted categorical. `order_out` (when given) receives the left bins in the rule's order.
__device__ FeatCand sorted_scan(const Ctx &c, const SplitCfgDev &cfg, const FeatDev &m, const int64_t *hist,
                                CatScratch &sc, uint8_t *order_out) {
    const int64_t *h = hist + 2 * static_cast<size_t>(m.hist_offset);
    const uint32_t lane = threadIdx.x & 63u;
    const int nb = static_cast<int>(m.num_bins < 256 ? m.num_bins : 256);
    // split.rs:740-760: bins with at least cat_smooth (estimated) rows, by (g / (h + cat_smooth), bin)
    bool ok[4];
    unsigned long long key[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = 1 + static_cast<int>(lane) + 64 * j;
        ok[j] = false;
        key[j] = 0;
        if (t < nb) {
            const double gu = static_cast<double>(h[2 * t]), hu = static_cast<double>(h[2 * t + 1]);
            ok[j] = static_cast<double>(bin_rows(c, hu)) >= cfg.cat_smooth;
            key[j] = total_order_bits((gu * c.scale_grad) / (hu * c.scale_hess + cfg.cat_smooth));
        }
        if (t < 256) {
            sc.key[t] = key[j];
            sc.eligible[t] = ok[j] ? 1 : 0;
        }
    }
    if (lane == 0) sc.eligible[0] = 0;
    int used = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) used += __popcll(__ballot(ok[j]));
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    // rank = eligible bins before this one in (key, bin) order
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = 1 + static_cast<int>(lane) + 64 * j;
        int rank = 0;
        if (ok[j])
            for (int u = 1; u < nb; ++u) {
                const unsigned long long ku = sc.key[u];
                rank += (sc.eligible[u] && (ku < key[j] || (ku == key[j] && u < t))) ? 1 : 0;
            }
        __builtin_amdgcn_wave_barrier();
        if (ok[j]) sc.order[rank] = static_cast<uint32_t>(t);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    FeatCand r = {};
    const int max_num_cat = static_cast<int>(cfg.max_cat_threshold < static_cast<uint64_t>((used + 1) / 2)
                                                 ? cfg.max_cat_threshold : static_cast<uint64_t>((used + 1) / 2));
    const int steps = used < max_num_cat ? used : max_num_cat;
    const double l2 = cfg.lambda_l2 + cfg.cat_l2;
    bool splittable = false;
    double fg = 0.0, bgn = 0.0, flg = 0.0, flh = 0.0, blg = 0.0, blh = 0.0;
    int fp = -1, bpz = -1;
    int64_t flc = 0, blc = 0;
    const bool ff = steps > 0 && sorted_run(c, cfg, h, sc, used, steps, true, l2, splittable, fg, fp, flg, flh, flc);
    const bool bf = steps > 0 && sorted_run(c, cfg, h, sc, used, steps, false, l2, splittable, bgn, bpz, blg, blh, blc);
    r.splittable = splittable ? 1 : 0;
    if (!ff && !bf) return r;
    const bool fwd = ff && !(bf && bgn > fg);  // split.rs:775-781: the backward run replaces only a lower gain
    const double gain = fwd ? fg : bgn;
    const int pos = fwd ? fp : bpz;
    const double ug = fwd ? flg : blg, uh = fwd ? flh : blh;
    r.found = 1;
    r.best_gain = gain;
    r.gain = gain - c.min_gain_shift;
    r.threshold = static_cast<uint32_t>(pos);
    r.left_grad = ug * c.scale_grad;
    r.left_hess = K_EPSILON + uh * c.scale_hess;
    r.left_count = fwd ? flc : blc;
    r.left_units_g = ug;
    r.left_units_h = uh;
    r.col = m.col;
    r.nan_idx = NO_BIN;
    r.rule = RULE_SORTED;
    r.cat_forward = fwd ? 1u : 0u;
    r.cat_count = static_cast<uint32_t>(pos + 1);
    for (int k = 0; k <= pos; ++k) {
        const uint32_t t = sc.order[fwd ? k : used - 1 - k];
        mask_set(r.cat_mask, t);
        if (order_out && lane == 0) order_out[k] = static_cast<uint8_t>(t);
    }
    return r;
}

// The candidate of a categorical feature (split.rs:847-862).
__device__ __forceinline__ FeatCand categorical_candidate(const Ctx &c, const SplitCfgDev &cfg, const FeatDev &m,
                                                          const int64_t *hist, CatScratch &sc, uint8_t *order_out) {
    if (m.num_bins <= cfg.max_cat_to_onehot) return onehot_scan(c, cfg, m, hist);
    return sorted_scan(c, cfg, m, hist, sc, order_out);
}

// split.rs:584-620 find_numerical (or a categorical search) for one feature of one leaf, by one wave. WIDE: the
// feature has two-byte bins (numerical, up to 1024); the kernels that scan them are instantiated apart, so the
// wide scan's registers do not lower the occupancy of the byte-bin scan.
template <bool WIDE>
__device__ FeatCand scan_feature(const Ctx &c, const SplitCfgDev &cfg, const FeatDev &m, const int64_t *hist, bool evaluate,
                                 CatScratch &sc, uint8_t *order_out) {
    if (!scan_searched(c, m, evaluate)) return FeatCand{};
    Grown rg = {}, fg = {};
    bool rf, ff;
    if constexpr (WIDE) {
        scan_numerical_wide(c, cfg, m, hist, rf, rg, ff, fg);
    } else {
        if (m.kind == 2) return categorical_candidate(c, cfg, m, hist, sc, order_out);
        scan_numerical(c, cfg, m, hist, rf, rg, ff, fg);
    }
    return feature_candidate(c, m, rf, rg, ff, fg);
}

// grid: (ceil(num_features / 4), num_jobs); 4 waves per block, a wave per feature.
template <bool WIDE>
__global__ __launch_bounds__(256) void k_split_scan(const ScanJob *__restrict__ jobs, const FeatDev *__restrict__ feats,
                                                    const uint8_t *__restrict__ evaluate, uint32_t num_features,
                                                    SplitCfgDev cfg, double sg, double sh,
                                                    uint8_t *cat_order /* [feature][256] or null */,
                                                    const DevScales *dsc /* when set: the scales */,
                                                    const uint8_t *skip = nullptr /* features k_split_scan_seg takes */) {
    if (dsc) {
        sg = dsc->sg;
        sh = dsc->sh;
    }
    __shared__ CatScratch cats[4];
    const ScanJob &job = jobs[blockIdx.y];
    uint32_t f = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (f >= num_features || (feats[f].wide != 0) != WIDE) return;  // the other instantiation's feature
    if (skip && skip[f]) return;
    Ctx c = make_ctx(cfg, sg, sh, job.units_grad, job.units_hess, job.count);
    FeatCand r = scan_feature<WIDE>(c, cfg, feats[f], job.hist, evaluate[f] != 0, cats[threadIdx.x >> 6],
                              cat_order ? cat_order + static_cast<size_t>(f) * 256 : nullptr);
    if ((threadIdx.x & 63) == 0) job.out[f] = r;
}

// k_split_scan for scan units of several numerical byte features of at most 64 bins (16 or 4 lanes a feature, as
// k_step_scan_seg): unit u holds unit_feat[u * UNIT_FEATS ...] (-1 padding), unit_segl[u] lanes each. A wave per
// unit and job. grid: (ceil(units / 4), jobs), 256 threads.
__global__ __launch_bounds__(256) void k_split_scan_seg(const ScanJob *__restrict__ jobs, const FeatDev *__restrict__ feats,
                                                        const uint8_t *__restrict__ evaluate, const int32_t *unit_feat,
                                                        const uint32_t *unit_segl, uint32_t units, SplitCfgDev cfg,
                                                        double sg, double sh) {
    const ScanJob &job = jobs[blockIdx.y];
    const uint32_t u = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
    if (u >= units) return;
    const uint32_t segl = unit_segl[u];  // 16 or 4, wave-uniform
    const int32_t f = unit_feat[u * UNIT_FEATS + lane / segl];
    const FeatDev m = f >= 0 ? feats[f] : FeatDev{};
    const Ctx c = make_ctx(cfg, sg, sh, job.units_grad, job.units_hess, job.count);
    Grown rg = {}, fg = {};
    bool rf = false, ff = false;
    if (segl == 16u) scan_numerical<16>(c, cfg, m, job.hist, rf, rg, ff, fg);
    else scan_numerical<4>(c, cfg, m, job.hist, rf, rg, ff, fg);
    FeatCand r = {};
    if (f >= 0 && scan_searched(c, m, evaluate[f] != 0)) r = feature_candidate(c, m, rf, rg, ff, fg);
    if ((lane & (segl - 1u)) == 0 && f >= 0) job.out[f] = r;
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
    uint32_t col, nan_idx;  // the feature's column-major index and NaN bin (NO_BIN: none)
    uint32_t rule;          // RULE_*: categorical rules send exactly the bins of cat_mask left
    uint32_t cat_count;
    uint32_t cat_mask[8];
};

// The best split over the per-feature candidates of `job` (highest gain, NaN as -inf, ties to the lower feature,
// split.rs:866-880) as the leaf's SplitOut (split.rs:631-651 finish), and its splittable flags. Block-wide (up
// to 1024 threads).
// split.rs:631-651 finish: the leaf's SplitInfo from its best feature's candidate.
__device__ __forceinline__ SplitOut split_out(const FeatCand &c, int f, const Ctx &x, const SplitCfgDev &cfg) {
    SplitOut o = {};
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
    const double l2 = c.rule == RULE_SORTED ? cfg.lambda_l2 + cfg.cat_l2 : cfg.lambda_l2;  // split.rs:667-680
    o.left_output = leaf_output(c.left_grad, c.left_hess, cfg.lambda_l1, l2);
    o.right_output = leaf_output(x.sum_grad - c.left_grad, x.sum_hess - c.left_hess, cfg.lambda_l1, l2);
    o.col = c.col;
    o.nan_idx = c.nan_idx;
    o.rule = c.rule;
    o.cat_count = c.cat_count;
    for (int w = 0; w < 8; ++w) o.cat_mask[w] = c.cat_mask[w];
    if (c.rule != RULE_NUMERICAL) {
        o.threshold = 0;
        o.default_left = 0;
    }
    return o;
}

__device__ void select_split(const ScanJob &job, int64_t count, uint32_t num_features, const SplitCfgDev &cfg, double sg,
                             double sh, SplitOut *out, uint8_t *splittable) {
    __shared__ double wgain[16];
    __shared__ int wfeat[16];
    const uint32_t nw = blockDim.x >> 6;
    double best = 0.0;
    int bf = -1;
    for (uint32_t f = threadIdx.x; f < num_features; f += blockDim.x) {
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
        for (uint32_t w = 1; w < nw; ++w)
            if (cand_better(wgain[w], wfeat[w], best, bf)) {
                best = wgain[w];
                bf = wfeat[w];
            }
        SplitOut o = {};
        if (bf >= 0) o = split_out(job.out[bf], bf, make_ctx(cfg, sg, sh, job.units_grad, job.units_hess, count), cfg);
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
// Device-driven growth (learner.rs:121-352) with speculative expansion.
//
// The reference grows leaf-wise: each split takes the leaf with the highest best gain (learner.rs:418-429), and
// a leaf's best split depends only on its own rows, its depth and its parent's splittable flags, never on when
// the leaf is split. So one split step here expands several leaves at once: the leaf the reference splits next
// (the blocker) and the highest-gain other leaves of the speculative tree. After each step, `advance` replays
// the reference's order over the gains known so far: it commits expansions while the leaf the reference splits
// next has been expanded (nodes and leaves get the reference's numbers), and plans the next step from the leaf
// where it stopped. Expansions the order has not reached when the tree is complete are dropped: their rows are
// merged back into ascending order (every leaf's rows are ascending, since the root's are and every partition
// is stable).
// ---------------------------------------------------------------------------------------------------------

// learner.rs:432-452 bin_split: word w of the bins that go left; numerical: bins 0..=threshold and the NaN bin when
// missing values go left; categorical: the rule's bins. A wide feature's split carries its rule instead (threshold,
// NaN bin + 1 when missing values go left; rule_left).
__device__ __forceinline__ uint32_t left_bins_word(const SplitOut &info, uint32_t w, uint32_t wide) {
    if (wide) {
        if (w == 0) return info.threshold;
        return w == 1 && info.default_left && info.nan_idx != NO_BIN ? info.nan_idx + 1u : 0u;
    }
    if (info.rule != RULE_NUMERICAL) return info.cat_mask[w];
    const uint32_t upto = info.threshold + 1;
    const uint32_t lo = 32 * w;
    uint32_t word = upto >= lo + 32 ? 0xffffffffu : (upto > lo ? (1u << (upto - lo)) - 1u : 0u);
    if (info.default_left && info.nan_idx != NO_BIN && (info.nan_idx >> 5) == w) word |= 1u << (info.nan_idx & 31u);
    return word;
}

constexpr uint32_t STEP_TILE = 4096;          // rows per partition tile: TILE_RPT per thread of a 1024-thread block
constexpr int TILE_RPT = STEP_TILE / 1024;
constexpr uint32_t CG_COLS = 4;               // slab columns per column group (k_step_reduce, k_step_scan)
// A split step's partials: workgroup b of a slab owns step_partial_stride(W) {g, h} pairs from pair b * stride,
// whether it writes 256 * W pairs or 256 * W packed words (a step can mix both). The stride is padded so that
// the same slot of consecutive partials does not fall at a power-of-two distance (which maps it to the same
// memory channel and bank).
constexpr uint32_t STEP_PARTIAL_PAD = 288;
__host__ __device__ constexpr size_t step_partial_stride(uint32_t w) { return 256u * static_cast<size_t>(w) + STEP_PARTIAL_PAD; }
constexpr uint32_t ST_AGG = 1, ST_INCL = 2;   // tile status: its own left count / lefts up to and including it
constexpr uint32_t LOOKBACK_SPINS = 1u << 20; // ~0.1 s of polling before a step gives up with an error

// Stripes of a job's `groups` partials that k_step_reduce adds on separate threads (combined through LDS), so that
// a thread adds about 8 partials (one round of loads): a power of two up to 32.
__device__ __forceinline__ uint32_t reduce_ways(uint32_t groups) {
    uint32_t w = 1;
    while (w < 32 && w * 8 < groups) w <<= 1;
    return w;
}

// Wave-wide sums of one value per lane: exclusive prefix and total.
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t v) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t x = __shfl_up(v, o);
        if (lane >= static_cast<uint32_t>(o)) v += x;
    }
    return v;
}
__device__ __forceinline__ uint32_t wave_excl_sum(uint32_t v) { return wave_incl_sum(v) - v; }
__device__ __forceinline__ uint32_t wave_total(uint32_t v) { return __shfl(wave_incl_sum(v), 63); }
__device__ __forceinline__ float wave_total_f32(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

constexpr uint32_t JMAX = 64;              // leaves expanded by one step at most (the plan's capacity)
// a step's jobs at most (GrowState::jcap): trees of up to LEAVES_SMALL leaves take 32, where a longer speculation
// mostly expands leaves the tree commits late or never; larger trees take JMAX, their steps being bound by the job count
__host__ __device__ constexpr uint32_t grow_jcap(uint32_t num_leaves) { return num_leaves <= LEAVES_SMALL ? 32u : JMAX; }
constexpr uint32_t SPEC_FEW = 8;           // at most this many: picked by repeated wave maxima (top_few)
constexpr uint32_t GROW_MAX_LEAVES = 2048;  // num_leaves of a device-grown tree at most
// Speculative leaves of a tree of num_leaves: 4 per leaf up to 512 leaves, then 2 per further leaf (the expansions
// a tree keeps need 2 per leaf; the rest is the room for speculating ahead, which advance keeps within it).
__host__ __device__ constexpr uint32_t grow_tcap(uint32_t num_leaves) {
    return num_leaves <= 512 ? 4 * num_leaves + 64 : 2 * num_leaves + 1088;
}

constexpr uint32_t T_LEAF = 0, T_PLANNED = 1, T_EXPANDED = 2;  // a speculative leaf's state

// A leaf of the speculative tree: the committed leaves and the children of every expansion.
struct TLeaf {
    uint32_t begin, count;   // rows in the partition
    double ug, uh;           // sums in histogram units
    int64_t cnt;             // exact row count
    int32_t slot;            // histogram slot, -1: none
    uint32_t has_best;
    uint32_t buf;            // partition buffer holding the rows
    uint32_t rev;            // the rows are stored last-first (right children of a split step)
    int32_t depth;
    uint32_t state;          // T_LEAF, T_PLANNED (expanded by the running step), T_EXPANDED
    int32_t kid;             // the children kid (left) and kid + 1 (right), once planned; -1 before
    uint32_t pad_;
    double value, weight;    // the leaf's output and hessian weight in the tree (from its parent's split)
    SplitOut best;
};

// The part of a speculative leaf that advance reads for every leaf, kept apart for one coalesced load.
struct TKey {
    double gain;  // best gain, when `has`
    uint32_t has;
    uint32_t state;
    int32_t kid;
    uint32_t pad_;
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
    uint32_t *left_bins;  // [node][8]: the bins that go left (BinSplit::left_bins)
    uint32_t *leaf_range; // [leaf][2]: the leaf's rows in the partition (begin, count)
};

// One leaf expanded by a split step (learner.rs:249-290): written by advance, read by the step's kernels.
struct JobPlan {
    uint32_t t;                   // the speculative leaf expanded
    uint32_t begin, count;        // its rows in the partition
    uint32_t col;                 // column-major index of the split feature
    uint32_t left_bins[8];
    uint32_t wide;                // left_bins hold a wide feature's numerical rule (rule_left)
    uint32_t built_side;          // 0: the left child is histogrammed, 1: the right (learner.rs:271-275)
    uint32_t hist;                // the built child is histogrammed (learner.rs:266-268)
    int32_t parent_slot, built_slot;
    uint32_t src_buf, src_rev;    // the buffer holding the leaf's rows (its children go to the other) and order
    uint32_t ntiles, tile_base;   // partition tiles and the first one's status word
    uint32_t groups, group_base;  // k_step_rows workgroups, one partial each
    uint32_t packed;              // the partials are packed 16/16 LDS words (one tile per workgroup)
    uint32_t ways;                // k_step_reduce stripes of the partials (reduce_ways)
    uint32_t red_base, red_items; // k_step_reduce work items: per column group, `ways` (packed) or 4 * `ways`
    uint32_t scan_base, scan_items;  // k_step_scan work items: a scan per column group (when histogrammed)
    uint32_t ticket;              // next partition tile to hand out
    uint32_t left;                // rows going left, written by the last tile
    int32_t kid;                  // the children's speculative leaves
    int64_t parent_count;
    double child_ug[2], child_uh[2];  // the children's sums in histogram units (left, right)
};

// A split step: the plan of step s is plans[s % 2], written by the step before it.
struct StepPlan {
    uint32_t njobs;
    uint32_t total_groups;  // k_step_rows workgroups in use
    uint32_t total_red;     // k_step_reduce work items
    uint32_t total_scan;    // k_step_scan work items
    uint32_t epoch;         // tags the step's tile status words
    uint32_t pad_[3];
    // the jobs' first workgroup, reduce item and scan item side by side (a job search reads one run of words)
    uint32_t group_base[JMAX], red_base[JMAX], scan_base[JMAX];
    JobPlan jobs[JMAX];
};

// The job whose range of work holds x: the last whose first element (bases[k]) is at or below it. The bases are read
// as one unrolled run, so the search is one round of loads: of the first 32 when the step has no more jobs (the
// whole run cost the latency-bound k_step_reduce 15% in such steps).
template <uint32_t N>
__device__ __forceinline__ uint32_t job_search(const uint32_t (&bases)[JMAX], uint32_t njobs, uint32_t x) {
    uint32_t j = 0;
#pragma unroll
    for (uint32_t k = 1; k < N; ++k)
        if (k < njobs && x >= bases[k]) j = k;
    return j;
}
__device__ __forceinline__ uint32_t job_of(const uint32_t (&bases)[JMAX], uint32_t njobs, uint32_t x) {
    return njobs <= 32u ? job_search<32>(bases, njobs, x) : job_search<JMAX>(bases, njobs, x);
}

struct GrowCtl {
    uint32_t num_leaves;   // committed leaves
    uint32_t done;         // no further step this tree
    uint32_t error;        // an invariant failed: 1 a child without rows, 3 a look-back gave up, 4 no room for a step
    uint32_t ntent;        // speculative leaves in use
    uint32_t next_slot;    // next free histogram slot
    uint32_t pending;      // expanded leaves not yet committed
    uint32_t epoch;        // split steps planned so far (kept across trees; tags tile status words)
    uint32_t steps;        // split steps planned this tree
    uint32_t expansions;   // leaves expanded this tree
    uint32_t pad_;
    uint32_t err_info[8];  // error 1: the job, its leaf, rows, left rows, tiles, workgroups, packed, jobs
    double hist_rows;      // rows histogrammed (built children), and rows x evaluated features
    double hist_bins;
    double hist_builds;    // child histograms built
    double part_rows;      // rows partitioned by the split steps
};

// Histogram slots: the root's is slot 0, each expansion that histograms takes the next free slot for its built
// child, and the other child keeps its parent's slot (a slot is never reused within a tree).
struct GrowState {
    GrowCtl *ctl;
    StepPlan *plans;          // [2]
    TLeaf *tl;                // [tcap], 0 is the root
    TKey *tk;                 // [tcap]
    int32_t *leaf_t;          // [num_leaves]: each committed leaf's speculative leaf
    uint8_t *leaf_left;       // [num_leaves]: the committed leaf is its parent's left child
    uint8_t *splittable;      // [tcap][nf]
    ScanJob *jobs;            // [1]: the root's search
    FeatCand *cands;          // [JMAX][2][nf]
    uint8_t *evaluate;        // [nf]: the root's evaluated features
    const uint8_t *mask;      // [nf], the tree's feature mask
    const FeatDev *feats;
    TreeDev tree;
    int64_t *pool;
    uint64_t slot_stride;
    uint32_t nf, num_leaves, sums_feature;
    uint32_t tcap, nslots;    // speculative leaves and histogram slots available
    int32_t max_depth;
    SplitCfgDev cfg;
    double sg, sh;
    const struct DevScales *dsc;  // when set, the scales are these (made on the device), not sg and sh
    uint32_t target_groups;   // k_step_rows workgroups a step is spread over
    uint32_t jcap;            // jobs a step at most: grow_jcap(num_leaves)
    uint32_t ncg;             // column groups of k_step_reduce
    uint32_t nsg;             // scan units of k_step_scan (a wave per unit and child)
    uint32_t flush_rows;      // rows a packed 16/16 LDS word can take
    uint32_t tile_cap;        // k_step_rows tiles a workgroup may take (its i32 sums of the quantized units)
    float hist_weight;        // the planner's cost of a tile of histogrammed rows, in partitioned tiles of a dense
    float sparse_weight;      // leaf, and the most a tile of a sparse leaf costs more
};

__device__ __forceinline__ double grow_sg(const GrowState &g) { return g.dsc ? g.dsc->sg : g.sg; }
__device__ __forceinline__ double grow_sh(const GrowState &g) { return g.dsc ? g.dsc->sh : g.sh; }

__device__ __forceinline__ bool depth_allows(const GrowState &g, int32_t d) { return g.max_depth <= 0 || d < g.max_depth; }

// Brings each listed run of rows into the first partition buffer in ascending order: copied from the second
// buffer (reversed when stored last-first), or reversed in place. grid: (x, runs).
struct RowRun {
    uint32_t begin, count, buf, rev;
};

__global__ void k_consolidate(const RowRun *__restrict__ runs, const uint32_t *__restrict__ buf1, uint32_t *__restrict__ buf0) {
    const RowRun l = runs[blockIdx.y];
    const uint32_t b = l.begin, n = l.count;
    const uint32_t stride = gridDim.x * blockDim.x;
    if (l.buf) {
        for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
            buf0[b + i] = buf1[l.rev ? b + n - 1 - i : b + i];
    } else if (l.rev) {
        for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n / 2; i += stride) {
            uint32_t x = buf0[b + i], y = buf0[b + n - 1 - i];
            buf0[b + i] = y;
            buf0[b + n - 1 - i] = x;
        }
    }
}

// A leaf whose expansion was dropped holds its rows as ascending runs (its speculative descendants' rows), which
// pairwise merge rounds bring back into one ascending run: in round t, runs 2m and 2m + 1 of the level-t runs (each
// the merge of 2^t consecutive original runs, its start starts[min(p << t, runs)]) become one, a row's place being
// its place in its run plus the rows below it in the partner run (a binary search; the rows of a leaf are distinct).
// ceil(log2(runs)) rounds, each moving every row once from `src` to `dst`, so a leaf costs its rows times the rounds,
// not times its runs. grid: (x, leaves).
struct MergeJob {
    uint32_t begin, count;
    uint32_t first, runs;  // the runs' starts (relative to begin) are starts[first, first + runs], then `count`
};

__global__ void k_merge_round(const MergeJob *__restrict__ jobs, const uint32_t *__restrict__ starts, uint32_t t,
                              const uint32_t *__restrict__ src, uint32_t *__restrict__ dst) {
    const MergeJob m = jobs[blockIdx.y];
    const uint32_t *s = starts + m.first;
    const uint32_t *leaf = src + m.begin;
    const uint32_t nr = (m.runs + (1u << t) - 1u) >> t;  // level-t runs
    auto start = [&](uint32_t p) { return s[min(p << t, m.runs)]; };
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < m.count; i += gridDim.x * blockDim.x) {
        uint32_t lo = 0, hi = nr;  // the run holding i: the last p with start(p) <= i
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) >> 1;
            if (start(mid) <= i) lo = mid;
            else hi = mid;
        }
        const uint32_t p = lo, q = p ^ 1u;
        const uint32_t v = leaf[i];
        uint32_t pos = i;
        if (q < nr) {
            uint32_t a = start(q), b = start(q + 1);  // rows of run q below v: the first position holding more
            const uint32_t base = a;
            while (a < b) {
                const uint32_t mid = (a + b) >> 1;
                if (leaf[mid] < v) a = mid + 1;
                else b = mid;
            }
            pos = start(p & ~1u) + (i - start(p)) + (a - base);
        }
        dst[m.begin + pos] = v;
    }
}

__global__ void k_copy_back(const MergeJob *__restrict__ jobs, const uint32_t *__restrict__ buf1, uint32_t *__restrict__ buf0) {
    const MergeJob m = jobs[blockIdx.y];
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < m.count; i += gridDim.x * blockDim.x)
        buf0[m.begin + i] = buf1[m.begin + i];
}

// The tree at its start: one leaf holding the root rows, its histogram in slot 0 when it is searched.
__global__ void k_grow_init(GrowState g, uint32_t root_begin, uint32_t root_count, int64_t root_cnt, uint32_t searched) {
    if (threadIdx.x == 0) {
        GrowCtl &c = *g.ctl;
        c.num_leaves = 1;
        c.done = searched ? 0u : 1u;
        c.error = 0;
        c.ntent = 1;
        c.next_slot = 1;
        c.pending = 0;
        c.steps = 0;
        c.expansions = 0;
        c.hist_rows = 0.0;
        c.hist_bins = 0.0;
        c.hist_builds = 0.0;
        c.part_rows = 0.0;
        TLeaf l = {};
        l.begin = root_begin;
        l.count = root_count;
        l.cnt = root_cnt;
        l.slot = searched ? 0 : -1;
        l.state = T_LEAF;
        l.kid = -1;
        g.tl[0] = l;
        g.tk[0] = TKey{0.0, 0u, T_LEAF, -1, 0u};
        g.leaf_t[0] = 0;
        g.leaf_left[0] = 0;
        g.tree.leaf_value[0] = 0.0;
        g.tree.leaf_weight[0] = 0.0;
        g.tree.leaf_count[0] = 0;
        g.tree.leaf_parent[0] = -1;
        g.tree.leaf_depth[0] = 0;
        g.tree.leaf_range[0] = root_begin;
        g.tree.leaf_range[1] = root_count;
        // both step plans empty until advance writes one: a step launched on an empty plan does nothing
        for (int k = 0; k < 2; ++k) {
            g.plans[k].njobs = 0;
            g.plans[k].total_groups = 0;
            g.plans[k].total_red = 0;
            g.plans[k].total_scan = 0;
        }
    }
}

// learner.rs:143-156: the root's sums from the sums feature's bins (split.rs:101-108), and its search job.
// The root's sums are those of one feature's bins taken in bin order as f64. Every bin and every partial sum is an
// integer of magnitude below 2^53 (rows times units stays below 2^48), so each of those additions is exact and the
// result is the exact integer sum, which the block adds in i64 and converts once. grid: 1, 256 threads.
__global__ __launch_bounds__(256) void k_root_prep(GrowState g) {
    __shared__ int64_t part[2][4];
    const TLeaf &l = g.tl[0];
    const int64_t *h = g.pool + (size_t)l.slot * g.slot_stride;
    for (uint32_t f = threadIdx.x; f < g.nf; f += blockDim.x) g.evaluate[f] = g.mask[f];
    const FeatDev m = g.feats[g.sums_feature];
    int64_t sg = 0, sh = 0;
    for (uint32_t b = threadIdx.x; b < m.num_bins; b += blockDim.x) {
        sg += h[2 * ((size_t)m.hist_offset + b)];
        sh += h[2 * ((size_t)m.hist_offset + b) + 1];
    }
    for (int o = 32; o > 0; o >>= 1) {
        sg += static_cast<int64_t>(__shfl_xor(static_cast<long long>(sg), o));
        sh += static_cast<int64_t>(__shfl_xor(static_cast<long long>(sh), o));
    }
    const uint32_t wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0) {
        part[0][wave] = sg;
        part[1][wave] = sh;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t tg = 0, th = 0;
        for (uint32_t w = 0; w < blockDim.x / 64; ++w) {
            tg += part[0][w];
            th += part[1][w];
        }
        const double dg = static_cast<double>(tg), dh = static_cast<double>(th);
        g.tl[0].ug = dg;
        g.tl[0].uh = dh;
        g.jobs[0] = ScanJob{h, dg, dh, l.cnt, g.cands};
    }
}

// ---------------------------------------------------------------------------------------------------------
// advance: the reference's order over the known gains, then the next step's plan. Block-wide (1024 threads);
// `scratch` is LDS of at least sizeof(AdvShared) bytes.
// ---------------------------------------------------------------------------------------------------------

template <uint32_t MAXL>
struct AdvShared {
    static constexpr uint32_t TCAP = grow_tcap(MAXL);
    static constexpr uint32_t CAND = (TCAP + 1) / 2 + 1;  // unexpanded leaves: E + 1 of the 2E + 1 of E expansions
    double gain[TCAP];                    // speculative leaves' best gains
    uint32_t meta[TCAP];                  // bit 0: has a best split; bits 1-2: state; bits 3..: kid + 1
    uint16_t leaf_t[MAXL];                // committed leaf -> speculative leaf, as the replay goes
    int16_t pnode[MAXL];                  // committed leaf -> the internal node above it (-1: the root)
    uint8_t is_left[MAXL];                // committed leaf is its node's left child
    uint8_t touched[MAXL];                // committed leaf changed by this replay
    // committed leaf's replay key (0: none): replay_key64 in trees of more than 512 leaves, where 32-bit keys meet
    // the winner's gain prefix often; replay_key<11> in the others, where its u32 wave max is the cheaper
    std::conditional_t<(MAXL > LEAVES_SMALL), uint64_t, uint32_t> key[MAXL];
    // trees of up to 512 leaves (replay_reg): an expanded speculative leaf's children, left then right, as their
    // replay_key<11> without the id bits (0: no key), bit 0 set when the child has a split and a NaN gain
    uint2 crec[MAXL > LEAVES_SMALL ? 1 : TCAP];
    uint32_t leaf_m[MAXL > LEAVES_SMALL ? MAXL : 1];  // trees of more than 512 leaves: committed leaf's s.meta word
    uint16_t ck[MAXL];                    // commit c: the speculative leaf split (node n0 - 1 + c)
    uint16_t cx[MAXL];                    // commit c: the leaf id split
    int16_t cpn[MAXL];                    // commit c: the split leaf's node above
    uint8_t cleft[MAXL];                  // commit c: the split leaf was its node's left child
    uint64_t ckey[CAND];                  // speculation candidates' keys (higher bound, gain, then lower leaf);
                                          // before them, frontier_bounds' parent links
    uint32_t crank[CAND];                 // and their ranks
    uint16_t cand[CAND];                  // speculation candidates
    uint16_t job_t[JMAX];
    uint64_t skey[JMAX];                  // select_top: the selected candidates' keys
    uint16_t scand[JMAX];                 // and leaves
    uint32_t ncand, ncommit, n, blocker, done, njobs, band, above, nsel, neligible;
    uint32_t nnan;                        // committed leaves whose best gain is NaN (replay_lds)
};

__device__ __forceinline__ uint32_t key_meta(const TKey &k) {
    return (k.has ? 1u : 0u) | (k.state << 1) | (static_cast<uint32_t>(k.kid + 1) << 3);
}

// A committed leaf's replay key: the top 32 - IDB bits of its positive gain (a positive double's bits order as its
// value), then the lower leaf id (2^IDB - 1 - id); 0 for a leaf without a split or a positive gain. One u32 max over
// the wave finds the highest key; it is best_leaf's choice unless another leaf shares its gain prefix, which the
// replay then settles on the exact gains. IDB = 9 takes trees of up to 512 leaves, 11 up to 2048.
template <int IDB>
__device__ __forceinline__ uint32_t replay_key(double gain, uint32_t meta, uint32_t id) {
    if (!(meta & 1u) || !(gain > 0.0)) return 0u;
    uint32_t p = static_cast<uint32_t>(__builtin_bit_cast(uint64_t, gain) >> (31 + IDB));
    p = p ? p : 1u;
    return (p << IDB) | ((1u << IDB) - 1u - id);
}

// replay_key in 64 bits for trees of up to 2048 leaves (replay_lds): the positive gain's bits without their low 11
// (its exponent and 41 bits of mantissa) above 2047 - leaf id. Two gains share that prefix only when they agree to
// about 5e-13 (32-bit keys kept 21 bits, and at 2047 leaves a third of the commits met a leaf with the winner's
// prefix, each settled by an exact f64 argmax).
__device__ __forceinline__ uint64_t replay_key64(double gain, uint32_t meta, uint32_t id) {
    if (!(meta & 1u) || !(gain > 0.0)) return 0ull;
    uint64_t p = __builtin_bit_cast(uint64_t, gain) >> 11;
    p = p ? p : 1ull;
    return (p << 11) | (2047u - id);
}

// replay_lds's key of a leaf, in the width of the key array (Key)
template <class Key>
__device__ __forceinline__ Key leaf_key(double gain, uint32_t meta, uint32_t id) {
    if constexpr (sizeof(Key) == 8) return replay_key64(gain, meta, id);
    else return replay_key<11>(gain, meta, id);
}

// The replay of advance (learner.rs:158-163 with best_leaf, learner.rs:418-429) on one wave. Lane l owns committed
// leaves l, l + 64, ... (NPL of them, NPL * 64 >= num_leaves); their state is in LDS (speculative leaf, node above,
// its state word, left and changed flags, and the replay key in s.key) and only the lane's largest key is in a
// register. A commit is one wave max of those (the reference's argmax only matters while the best gain is positive:
// otherwise the tree stops), with an exact f64 argmax only when two leaves share the winner's gain prefix: a lane
// other than the winner's holds such a key exactly when its largest key has the prefix, and the winner's own keys
// are read from s.key by NPL lanes at once, with the winner's state, and serve again for that lane's new largest key
// after the commit. So a commit waits on two LDS reads: those, then its children's gains and state words. The rule
// that the first leaf with a split decides when its gain is NaN takes a wave minimum, only while some leaf has a NaN
// gain (they are counted). Leaves the commits, the committed-leaf arrays and the outcome in `s`.
template <int NPL, typename S>
__device__ __forceinline__ void replay_lds(S &s, uint32_t n0, uint32_t L) {
    constexpr int IDB = 11;
    static_assert(NPL * 64 <= (1 << IDB) && NPL * 64 <= static_cast<int>(GROW_MAX_LEAVES) && NPL <= 64, "leaf ids fit");
    constexpr uint64_t IDM = (1u << IDB) - 1u;
    static_assert(sizeof(s.leaf_m) >= sizeof(uint32_t) * NPL * 64, "the committed leaves' state words");
    using Key = std::remove_cv_t<std::remove_reference_t<decltype(s.key[0])>>;
    constexpr bool K64 = sizeof(Key) == 8;
    auto key_of = [](double gain, uint32_t meta, uint32_t id) -> Key { return leaf_key<Key>(gain, meta, id); };
    auto wave_max_key = [](Key v) -> Key {  // 64-bit keys: two gains share the high word when within about 1e-6
        if constexpr (K64) return wave_max_u64_hi(v);
        else return wave_max_u32(v);
    };
    const uint32_t lane = threadIdx.x & 63u;
    // the keys (0 past the committed leaves) and the NaN count were made by the whole block (advance)
    Key lk = 0;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        const Key key = s.key[lane + 64u * j];
        lk = key > lk ? key : lk;
    }
    uint32_t nan_leaves = s.nnan;
    uint32_t n = n0, nc = 0, blocker = 0;
    bool done = false;
    for (;;) {
        if (n >= L) {
            done = true;
            break;
        }
        // best_leaf: the first leaf with a split decides when its gain is NaN (nothing beats NaN under `>`)
        if (nan_leaves) {
            int lfirst = 1 << 30;
            for (int j = NPL - 1; j >= 0; --j) {  // descending, so the lowest id is the one kept
                const uint32_t id = lane + 64u * j;
                if (id >= n) continue;
                const uint32_t t = s.leaf_t[id];
                const double gj = s.gain[t];
                if (s.meta[t] & 1u) lfirst = 2 * static_cast<int>(id) + (gj != gj ? 1 : 0);
            }
            const int first = wave_min_i32(lfirst);
            if (first < (1 << 30) && (first & 1)) {
                done = true;
                break;
            }
        }
        const Key best = wave_max_key(lk);
        if (best == 0u) {
            done = true;
            break;
        }
        uint32_t x = static_cast<uint32_t>(IDM - (best & IDM));
        // the winner's lane's keys (0 past the leaves) and the winner's state, read together
        Key kk = lane < static_cast<uint32_t>(NPL) ? s.key[(x & 63u) + 64u * lane] : Key{0};
        uint32_t k = s.leaf_t[x], m = s.leaf_m[x];
        int32_t pn = s.pnode[x];
        uint32_t xl = s.is_left[x];
        {  // another leaf with the winner's gain prefix: the exact gains decide (then the lower id)
            const Key bp = best >> IDB;
            const bool other = (lane != (x & 63u) && (lk >> IDB) == bp) || ((kk >> IDB) == bp && kk != best);
            if (__ballot(other)) {
                double kg = 0.0;
                int ki = -1;
                for (int j = NPL - 1; j >= 0; --j) {  // descending, so the lowest id is kept on equal gains
                    const uint32_t id = lane + 64u * j;
                    if ((s.key[id] >> IDB) != bp) continue;
                    const double gj = s.gain[s.leaf_t[id]];
                    if (ki < 0 || gj >= kg) {
                        kg = gj;
                        ki = static_cast<int>(id);
                    }
                }
                wave_argmax(kg, ki);
                x = static_cast<uint32_t>(ki);
                kk = lane < static_cast<uint32_t>(NPL) ? s.key[(x & 63u) + 64u * lane] : Key{0};
                k = s.leaf_t[x];
                m = s.leaf_m[x];
                pn = s.pnode[x];
                xl = s.is_left[x];
            }
        }
        if (((m >> 1) & 3u) != T_EXPANDED) {
            blocker = k;
            break;
        }
        const uint32_t kid = (m >> 3) - 1u;
        const double g0 = s.gain[kid], g1 = s.gain[kid + 1];
        const uint32_t m0 = s.meta[kid], m1 = s.meta[kid + 1];
        const Key k0 = key_of(g0, m0, x), k1 = key_of(g1, m1, n);
        // leaf x becomes the left child, leaf n the right one, both under node n - 1
        const int32_t node = static_cast<int32_t>(n) - 1;
        if (lane == 0) {
            s.ck[nc] = static_cast<uint16_t>(k);
            s.cx[nc] = static_cast<uint16_t>(x);
            s.cpn[nc] = static_cast<int16_t>(pn);
            s.cleft[nc] = static_cast<uint8_t>(xl);
            s.leaf_t[x] = static_cast<uint16_t>(kid);
            s.leaf_m[x] = m0;
            s.pnode[x] = static_cast<int16_t>(node);
            s.is_left[x] = 1;
            s.touched[x] = 1;
            s.key[x] = k0;
            s.leaf_t[n] = static_cast<uint16_t>(kid + 1);
            s.leaf_m[n] = m1;
            s.pnode[n] = static_cast<int16_t>(node);
            s.is_left[n] = 0;
            s.touched[n] = 1;
            s.key[n] = k1;
        }
        nan_leaves += ((m0 & 1u) && g0 != g0 ? 1u : 0u) + ((m1 & 1u) && g1 != g1 ? 1u : 0u);
        // the lanes' largest keys: x's lane (its largest was x's old key) from its keys as read, with x's key now k0
        // (and n's k1 when n is in that lane); n's lane takes k1 as well
        const uint32_t lx = x & 63u, ln = n & 63u;
        Key kv = lane == (x >> 6) ? k0 : kk;
        kv = ln == lx && lane == (n >> 6) ? k1 : kv;
        const Key mx = wave_max_key(kv);
        if (lane == lx) lk = mx;
        else if (lane == ln) lk = k1 > lk ? k1 : lk;
        ++nc;
        ++n;
    }
    if (lane == 0) {
        s.ncommit = nc;
        s.n = n;
        s.done = done ? 1u : 0u;
        s.blocker = blocker;
    }
}

// replay_lds for trees of up to 512 leaves (NPL 4 or 8) with the replay keys and speculative leaves of lane l's
// committed leaves (l, l + 64, ...) in its registers: the test for another leaf with the winner's gain prefix
// needs no LDS, the winner's speculative leaf is a read of its lane, and its children's keys come from one read
// of s.crec (their key prefixes, made by the whole block), so a commit waits on one LDS read (that record with the
// state word) where replay_lds waits on five. Lane 0 keeps the committed-leaf arrays in LDS up to date for
// apply_commits and the NaN rule, which reads them; s.key is left as the block made it.
template <int NPL, typename S>
__device__ __forceinline__ void replay_reg(S &s, uint32_t n0, uint32_t L) {
    constexpr int IDB = 11;
    static_assert(NPL * 64 <= static_cast<int>(LEAVES_SMALL) && sizeof(s.key[0]) == 4, "u32 keys of 512 leaves at most");
    constexpr uint32_t IDM = (1u << IDB) - 1u;
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t rk[NPL], rt[NPL], lk = 0;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {  // keys are 0 past the committed leaves, whose speculative leaf is then unused
        const uint32_t id = lane + 64u * j;
        rk[j] = s.key[id];
        rt[j] = s.leaf_t[id];
        lk = rk[j] > lk ? rk[j] : lk;
    }
    uint32_t nan_leaves = s.nnan;
    uint32_t n = n0, nc = 0, blocker = 0;
    bool done = false;
    for (;;) {
        if (n >= L) {
            done = true;
            break;
        }
        // best_leaf: the first leaf with a split decides when its gain is NaN (nothing beats NaN under `>`)
        if (nan_leaves) {
            int lfirst = 1 << 30;
            for (int j = NPL - 1; j >= 0; --j) {  // descending, so the lowest id is the one kept
                const uint32_t id = lane + 64u * j;
                if (id >= n) continue;
                const uint32_t t = s.leaf_t[id];
                const double gj = s.gain[t];
                if (s.meta[t] & 1u) lfirst = 2 * static_cast<int>(id) + (gj != gj ? 1 : 0);
            }
            const int first = wave_min_i32(lfirst);
            if (first < (1 << 30) && (first & 1)) {
                done = true;
                break;
            }
        }
        const uint32_t best = wave_max_u32(lk);
        if (best == 0u) {
            done = true;
            break;
        }
        uint32_t x = IDM - (best & IDM);
        {  // another leaf with the winner's gain prefix: the exact gains decide (then the lower id)
            const uint32_t bp = best >> IDB;
            bool other = false;
            if (lane == (x & 63u)) {
#pragma unroll
                for (int j = 0; j < NPL; ++j) other = other || (rk[j] != best && (rk[j] >> IDB) == bp);
            } else {
                other = (lk >> IDB) == bp;
            }
            if (__ballot(other)) {
                double kg = 0.0;
                int ki = -1;
#pragma unroll
                for (int j = NPL - 1; j >= 0; --j) {  // descending, so the lowest id is kept on equal gains
                    if ((rk[j] >> IDB) != bp) continue;
                    const double gj = s.gain[rt[j]];
                    if (ki < 0 || gj >= kg) {
                        kg = gj;
                        ki = static_cast<int>(lane + 64u * j);
                    }
                }
                wave_argmax(kg, ki);
                x = static_cast<uint32_t>(ki);
            }
        }
        const uint32_t jx = x >> 6, lx = x & 63u, jn = n >> 6, ln = n & 63u;
        uint32_t tv = rt[0];
#pragma unroll
        for (int j = 1; j < NPL; ++j) tv = jx == static_cast<uint32_t>(j) ? rt[j] : tv;
        const uint32_t k = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(tv), static_cast<int>(lx)));
        const uint32_t m = s.meta[k];
        const uint2 c = s.crec[k];
        const int32_t pn = s.pnode[x];
        const uint32_t xl = s.is_left[x];
        if (((m >> 1) & 3u) != T_EXPANDED) {
            blocker = k;
            break;
        }
        const uint32_t kid = (m >> 3) - 1u;
        const uint32_t k0 = (c.x >> IDB) ? ((c.x & ~IDM) | (IDM - x)) : 0u;
        const uint32_t k1 = (c.y >> IDB) ? ((c.y & ~IDM) | (IDM - n)) : 0u;
        // leaf x becomes the left child, leaf n the right one, both under node n - 1
        const int32_t node = static_cast<int32_t>(n) - 1;
        if (lane == 0) {
            s.ck[nc] = static_cast<uint16_t>(k);
            s.cx[nc] = static_cast<uint16_t>(x);
            s.cpn[nc] = static_cast<int16_t>(pn);
            s.cleft[nc] = static_cast<uint8_t>(xl);
            s.leaf_t[x] = static_cast<uint16_t>(kid);
            s.pnode[x] = static_cast<int16_t>(node);
            s.is_left[x] = 1;
            s.touched[x] = 1;
            s.leaf_t[n] = static_cast<uint16_t>(kid + 1);
            s.pnode[n] = static_cast<int16_t>(node);
            s.is_left[n] = 0;
            s.touched[n] = 1;
        }
        nan_leaves += (c.x & 1u) + (c.y & 1u);
        uint32_t nk = 0;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            if (jx == static_cast<uint32_t>(j) && lane == lx) {
                rk[j] = k0;
                rt[j] = kid;
            }
            if (jn == static_cast<uint32_t>(j) && lane == ln) {
                rk[j] = k1;
                rt[j] = kid + 1u;
            }
            nk = rk[j] > nk ? rk[j] : nk;
        }
        lk = nk;
        ++nc;
        ++n;
    }
    if (lane == 0) {
        s.ncommit = nc;
        s.n = n;
        s.done = done ? 1u : 0u;
        s.blocker = blocker;
    }
}

// The replay of replay_lds for trees of up to 128 leaves (NPL 1 or 2), where registers beat LDS: lane l holds committed
// leaves l, l + 64, ... (NPL of them, NPL * 64 >= num_leaves) in registers (replay key, meta, speculative leaf, node
// above, left / has-split / NaN-gain flags). A commit is one u32 wave max of the keys (the reference's argmax only
// matters while the best gain is positive: otherwise the tree stops), with an exact f64 argmax only when two
// leaves share the winner's gain prefix; the rule that the first leaf with a split decides when its gain is NaN
// takes a wave minimum, only while some leaf has a NaN gain. Leaves the commits, the committed-leaf arrays and the
// outcome in `s`.
template <int NPL, typename S>
__device__ __forceinline__ void replay(S &s, uint32_t n0, uint32_t L) {
    constexpr int IDB = 9;
    static_assert(NPL * 64 <= (1 << IDB), "leaf ids fit the key");
    constexpr uint32_t IDM = (1u << IDB) - 1u;
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t rk[NPL], rm[NPL], rt[NPL];
    int32_t rp[NPL];
    uint32_t rl = 0, rtouch = 0, rhas = 0, rnan = 0;  // bit j: leaf lane + 64 j is a left child / changed / ...
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        const uint32_t id = lane + 64u * j;
        rk[j] = 0;
        rm[j] = 0;
        rt[j] = 0;
        rp[j] = -1;
        if (id < n0) {
            rt[j] = s.leaf_t[id];
            const double gj = s.gain[rt[j]];
            rm[j] = s.meta[rt[j]];
            rk[j] = replay_key<IDB>(gj, rm[j], id);
            rp[j] = s.pnode[id];
            rl |= s.is_left[id] ? 1u << j : 0u;
            rhas |= (rm[j] & 1u) ? 1u << j : 0u;
            rnan |= (rm[j] & 1u) && gj != gj ? 1u << j : 0u;
        }
    }
    uint32_t n = n0, nc = 0, blocker = 0;
    bool done = false;
    for (;;) {
        if (n >= L) {
            done = true;
            break;
        }
        // best_leaf: the first leaf with a split decides when its gain is NaN (nothing beats NaN under `>`)
        if (__ballot(rnan != 0u)) {
            int lfirst = 1 << 30;
#pragma unroll
            for (int j = NPL - 1; j >= 0; --j)  // descending, so the lowest id is the one kept
                if ((rhas >> j) & 1u) lfirst = 2 * static_cast<int>(lane + 64u * j) + static_cast<int>((rnan >> j) & 1u);
            const int first = wave_min_i32(lfirst);
            if (first < (1 << 30) && (first & 1)) {
                done = true;
                break;
            }
        }
        // otherwise the first highest gain among the rest (a NaN later never wins); none positive ends the tree
        uint32_t lk = 0;
#pragma unroll
        for (int j = 0; j < NPL; ++j) lk = rk[j] > lk ? rk[j] : lk;
        const uint32_t best = wave_max_u32(lk);
        if (best == 0u) {
            done = true;
            break;
        }
        uint32_t x = IDM - (best & IDM);
        {  // another leaf with the winner's gain prefix: the exact gains decide (then the lower id)
            const uint32_t bp = best >> IDB;
            uint32_t same = 0;
#pragma unroll
            for (int j = 0; j < NPL; ++j) same += (rk[j] >> IDB) == bp && rk[j] != best ? 1u : 0u;
            if (__ballot(same != 0u)) {
                double kg = 0.0;
                int ki = -1;
#pragma unroll
                for (int j = NPL - 1; j >= 0; --j) {  // descending, so the lowest id is kept on equal gains
                    if ((rk[j] >> IDB) != bp) continue;
                    const double gj = s.gain[rt[j]];
                    if (ki < 0 || gj >= kg) {
                        kg = gj;
                        ki = static_cast<int>(lane + 64u * j);
                    }
                }
                wave_argmax(kg, ki);
                x = static_cast<uint32_t>(ki);
            }
        }
        const uint32_t jx = x >> 6, lx = x & 63u;
        // jx is wave-uniform: indexed register reads
        const uint32_t vm = rm[jx], vt = rt[jx];
        const int32_t vp = rp[jx];
        const uint32_t m = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(vm), lx));
        const uint32_t k = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(vt), lx));
        if (((m >> 1) & 3u) != T_EXPANDED) {
            blocker = k;
            break;
        }
        const int32_t pn = __builtin_amdgcn_readlane(vp, lx);
        const uint32_t xl = (static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(rl), lx)) >> jx) & 1u;
        const uint32_t kid = (m >> 3) - 1u;
        const double g0 = s.gain[kid], g1 = s.gain[kid + 1];
        const uint32_t m0 = s.meta[kid], m1 = s.meta[kid + 1];
        if (lane == 0) {
            s.ck[nc] = static_cast<uint16_t>(k);
            s.cx[nc] = static_cast<uint16_t>(x);
            s.cpn[nc] = static_cast<int16_t>(pn);
            s.cleft[nc] = static_cast<uint8_t>(xl);
        }
        // leaf x becomes the left child, leaf n the right one, both under node n - 1
        const int32_t node = static_cast<int32_t>(n) - 1;
        const uint32_t jn = n >> 6, ln = n & 63u;
        // (jx and jn are wave-uniform: indexed register moves, one slot each)
        if (lane == lx) {
            rt[jx] = kid;
            rk[jx] = replay_key<IDB>(g0, m0, x);
            rm[jx] = m0;
            rp[jx] = node;
        }
        if (lane == ln) {
            rt[jn] = kid + 1;
            rk[jn] = replay_key<IDB>(g1, m1, n);
            rm[jn] = m1;
            rp[jn] = node;
        }
        const uint32_t bx = 1u << jx, bn = 1u << jn;
        if (lane == lx) {
            rl |= bx;
            rtouch |= bx;
            rhas = (rhas & ~bx) | ((m0 & 1u) ? bx : 0u);
            rnan = (rnan & ~bx) | ((m0 & 1u) && g0 != g0 ? bx : 0u);
        }
        if (lane == ln) {
            rl &= ~bn;
            rtouch |= bn;
            rhas = (rhas & ~bn) | ((m1 & 1u) ? bn : 0u);
            rnan = (rnan & ~bn) | ((m1 & 1u) && g1 != g1 ? bn : 0u);
        }
        ++nc;
        ++n;
    }
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        const uint32_t id = lane + 64u * j;
        if (id < n) {
            s.leaf_t[id] = static_cast<uint16_t>(rt[j]);
            s.pnode[id] = static_cast<int16_t>(rp[j]);
            s.is_left[id] = static_cast<uint8_t>((rl >> j) & 1u);
            s.touched[id] = static_cast<uint8_t>((rtouch >> j) & 1u);
        }
    }
    if (lane == 0) {
        s.ncommit = nc;
        s.n = n;
        s.done = done ? 1u : 0u;
        s.blocker = blocker;
    }
}

// The `spec` highest of the `ncand` candidate keys s.ckey (distinct 64-bit keys) into s.job_t[1 .. spec], in key
// order, by a radix selection over the keys' 64 bits, 8 at a time from the top: a 256-bucket count of the
// candidates that still match the prefix found so far, the bucket where the count from the top reaches what is
// left to take, and the candidates above it taken. Every key is distinct, so after at most 8 rounds the prefix
// is a whole key. Block-wide; s.crank holds the counts.
// The `spec` highest candidate keys for a few expansions (spec <= SPEC_FEW), on one wave: `spec` rounds of a wave
// maximum over the keys not yet taken, each lane holding candidates lane, lane + 64, ... (at most 64 of them, a bit
// each in `taken`). The keys are distinct (they end in the leaf), so round r finds the key ranked r: jobs 1 .. spec in
// descending key order, as the ranking orders them.
template <typename S>
__device__ __forceinline__ void top_few(S &s, uint32_t ncand, uint32_t spec) {
    static_assert(S::CAND <= 64u * 64u, "a lane's candidates fit the taken mask");
    const uint32_t lane = threadIdx.x & 63u;
    uint64_t taken = 0;
    for (uint32_t r = 0; r < spec; ++r) {
        uint64_t best = 0;
        uint32_t at = 0;
        uint32_t q = 0;
        for (uint32_t i = lane; i < ncand; i += 64u, ++q) {
            const uint64_t k = s.ckey[i];
            if (!((taken >> q) & 1ull) && k > best) {
                best = k;
                at = i;
            }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const uint64_t ob = __shfl_xor(best, o);
            const uint32_t oa = static_cast<uint32_t>(__shfl_xor(static_cast<int>(at), o));
            if (ob > best) {
                best = ob;
                at = oa;
            }
        }
        // every candidate key is nonzero (a positive gain's bits), so the winner is a real candidate
        if ((at & 63u) == lane) taken |= 1ull << (at >> 6);
        if (lane == 0) s.job_t[1 + r] = s.cand[at];
    }
}

template <uint32_t MAXL>
__device__ void select_top(AdvShared<MAXL> &s, uint32_t ncand, uint32_t spec) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, nt = blockDim.x;
    uint32_t *count = s.crank;  // 256 buckets
    uint64_t prefix = 0, mask = 0;  // the bits fixed so far
    uint32_t taken = 0;             // candidates above the prefix, all taken
    if (tid == 0) s.nsel = 0;
    for (int shift = 56; shift >= 0 && taken < spec; shift -= 8) {
        for (uint32_t i = tid; i < 256u; i += nt) count[i] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < ncand; i += nt) {
            const uint64_t k = s.ckey[i];
            if ((k & mask) == prefix) atomicAdd(&count[static_cast<uint32_t>(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) {  // lane l: buckets 255 - 4 l down to 252 - 4 l
            uint32_t c = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) c += count[255u - 4u * lane - static_cast<uint32_t>(q)];
            const uint32_t incl = wave_incl_sum(c), before = incl - c;
            const unsigned long long hit = __ballot(taken + incl >= spec);
            if (lane == static_cast<uint32_t>(__builtin_ctzll(hit))) {  // the total reaches it: some lane hits
                uint32_t above = before, b = 255u - 4u * lane;
                for (int q = 0; q < 4; ++q, --b) {
                    if (taken + above + count[b] >= spec) break;
                    above += count[b];
                }
                s.band = b;
                s.above = above;
            }
        }
        __syncthreads();
        const uint32_t b = s.band, above = s.above, cb = count[b];  // read before the counts are cleared again
        // every matching candidate above bucket b is in
        for (uint32_t i = tid; i < ncand; i += nt) {
            const uint64_t k = s.ckey[i];
            if ((k & mask) == prefix && (static_cast<uint32_t>(k >> shift) & 255u) > b) {
                const uint32_t at = atomicAdd(&s.nsel, 1u);
                s.skey[at] = k;
                s.scand[at] = s.cand[i];
            }
        }
        taken += above;
        prefix |= static_cast<uint64_t>(b) << shift;
        mask |= uint64_t(255) << shift;
        __syncthreads();
        if (taken + cb == spec) {  // uniform: bucket b completes the selection (always so once the key is whole)
            for (uint32_t i = tid; i < ncand; i += nt) {
                const uint64_t k = s.ckey[i];
                if ((k & mask) == prefix) {
                    const uint32_t at = atomicAdd(&s.nsel, 1u);
                    s.skey[at] = k;
                    s.scand[at] = s.cand[i];
                }
            }
            taken = spec;
            __syncthreads();
        }
    }
    if (tid < spec) {  // the selected ones in key order
        const uint64_t ki = s.skey[tid];
        uint32_t rank = 0;
        for (uint32_t j = 0; j < spec; ++j) rank += s.skey[j] > ki ? 1u : 0u;
        s.job_t[1 + rank] = s.scand[tid];
    }
}

// The commits applied to the tree (tree.rs:143-177) by waves w0 .. w0 + nw - 1 of the block (nw >= 2): wave w0
// writes the new nodes and then, once they have landed, the links into nodes split again (a later commit of the step
// may split a leaf a node of the same step points to); the other waves write the changed leaves.
template <uint32_t MAXL>
__device__ void apply_commits(const GrowState &g, const AdvShared<MAXL> &s, uint32_t n0, uint32_t nc, uint32_t n,
                              uint32_t w0, uint32_t nw) {
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const TreeDev &t = g.tree;
    if (wave == w0) {
        for (uint32_t c = lane; c < nc; c += 64u) {
            const TLeaf &p = g.tl[s.ck[c]];
            const SplitOut &info = p.best;
            const uint32_t node = n0 - 1 + c;
            t.split_feature[node] = info.feature;
            const uint32_t wide = g.feats[info.feature].wide;
#pragma unroll
            for (uint32_t w = 0; w < 8; ++w) t.left_bins[static_cast<size_t>(node) * 8 + w] = left_bins_word(info, w, wide);
            t.split_gain[node] = static_cast<float>(info.gain + g.cfg.min_gain_to_split);
            t.threshold_bin[node] = info.threshold;
            t.default_left[node] = static_cast<uint8_t>(info.default_left);
            t.left_child[node] = ~static_cast<int32_t>(s.cx[c]);
            t.right_child[node] = ~static_cast<int32_t>(n0 + c);
            t.internal_weight[node] = p.weight;
            t.internal_value[node] = p.value;
            t.internal_count[node] = p.cnt;
        }
        __builtin_amdgcn_s_waitcnt(0);  // the nodes' children have landed before the links overwrite some
        for (uint32_t c = lane; c < nc; c += 64u) {
            const int32_t pn = s.cpn[c];
            if (pn < 0) continue;
            if (s.cleft[c]) t.left_child[pn] = static_cast<int32_t>(n0 - 1 + c);
            else t.right_child[pn] = static_cast<int32_t>(n0 - 1 + c);
        }
        return;
    }
    if (wave <= w0 || wave >= w0 + nw) return;
    for (uint32_t id = (wave - w0 - 1) * 64u + lane; id < n; id += (nw - 1) * 64u) {
        if (!s.touched[id]) continue;
        const uint32_t k = s.leaf_t[id];
        const TLeaf &l = g.tl[k];
        t.leaf_value[id] = l.value;
        t.leaf_weight[id] = l.weight;
        t.leaf_count[id] = l.cnt;
        t.leaf_parent[id] = s.pnode[id];
        t.leaf_depth[id] = l.depth;
        t.leaf_range[2 * id] = l.begin;
        t.leaf_range[2 * id + 1] = l.count;
        g.leaf_t[id] = static_cast<int32_t>(k);
        g.leaf_left[id] = s.is_left[id];
    }
}

// Each speculative leaf's bound after the replay: the smallest gain (as f32) on its path from the committed leaf
// above it (that leaf included) down to it, the order in which best_leaf would reach it (a leaf is committed before
// another whose bound is lower, since every leaf on its path must be committed first and each is the largest gain
// when it is). Into the .x half of each leaf's s.gain word (the replay's exact gains are no longer read), the leaf's
// gain as f32 in .y; leaves not below a committed leaf (the committed tree's nodes) get -1. Pointer jumping over
// parent links kept in the s.ckey words: a leaf's link is its parent until it meets a committed leaf, each round
// takes the minimum with its link's and doubles the link's reach, so ceil(log2(depth)) + 1 rounds end it (at most
// 16, which covers any tree of the sizes here). Block-wide.
template <uint32_t MAXL>
__device__ void frontier_bounds(AdvShared<MAXL> &s, uint32_t ntent, uint32_t n) {
    constexpr uint32_t PER = (AdvShared<MAXL>::TCAP + 511) / 512;  // leaves a thread (blocks of at least 512)
    constexpr uint32_t NONE = 0xffffu, UNDER = 1u << 16;             // link: bits 0-15; bit 16: below a committed leaf
    static_assert(AdvShared<MAXL>::TCAP < NONE, "leaf links fit 16 bits");
    static_assert(sizeof(s.ckey) >= sizeof(uint32_t) * AdvShared<MAXL>::TCAP, "the links fit the key words");
    uint32_t *link = reinterpret_cast<uint32_t *>(s.ckey);
    float2 *bw = reinterpret_cast<float2 *>(s.gain);
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    for (uint32_t k = tid; k < ntent; k += nt) link[k] = NONE;
    __syncthreads();
    for (uint32_t k = tid; k < ntent; k += nt) {
        const uint32_t m = s.meta[k];
        const double gk = s.gain[k];
        if (((m >> 1) & 3u) != T_LEAF && (m >> 3) != 0u) {  // expanded or planned: its children are kid, kid + 1
            const uint32_t kid = (m >> 3) - 1u;
            link[kid] = k;
            link[kid + 1] = k;
        }
        const float gf = (m & 1u) && gk == gk ? static_cast<float>(gk) : -1.0f;
        bw[k] = make_float2(gf, gf);  // read after the barrier below
    }
    __syncthreads();
    for (uint32_t id = tid; id < n; id += nt) link[s.leaf_t[id]] = UNDER | NONE;  // the committed leaves: the path's top
    __syncthreads();
    for (int round = 0; round < 16; ++round) {
        uint32_t nl[PER];
        float nb[PER];
        bool moved = false;
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i) {
            const uint32_t k = tid + nt * i;
            nl[i] = NONE;
            nb[i] = 0.0f;
            if (k >= ntent) continue;
            const uint32_t l = link[k];
            nl[i] = l;
            nb[i] = bw[k].x;
            if ((l & NONE) != NONE) {
                const uint32_t u = l & NONE, lu = link[u];
                nb[i] = fminf(nb[i], bw[u].x);
                nl[i] = (l & UNDER) | (lu & UNDER) | (lu & NONE);
                moved = true;
            }
        }
        const bool any = __syncthreads_or(moved ? 1 : 0) != 0;
#pragma unroll
        for (uint32_t i = 0; i < PER; ++i) {
            const uint32_t k = tid + nt * i;
            if (k < ntent) {
                link[k] = nl[i];
                bw[k].x = nb[i];
            }
        }
        __syncthreads();
        if (!any) break;
    }
    for (uint32_t k = tid; k < ntent; k += nt)
        if (!(link[k] & UNDER)) bw[k].x = -1.0f;
    __syncthreads();
}

// The bits of the R-th highest bound (frontier_bounds, positive f32 bits order as the values) among the leaves the
// tree may still commit: the unexpanded leaves with a split and a positive gain (the blocker among them) and the
// expanded ones not yet committed; 0 when there are fewer than R of them. best_leaf commits a leaf before any of
// lower bound, so a leaf below this bound is not among the next R commits and expanding it now is wasted. A radix
// selection over the bound bits, 8 at a time from the top (s.crank: 256 counts). Block-wide.
template <uint32_t MAXL>
__device__ uint32_t pool_threshold(AdvShared<MAXL> &s, uint32_t ntent, uint32_t R) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, nt = blockDim.x;
    const float2 *bw = reinterpret_cast<const float2 *>(s.gain);
    uint32_t *count = s.crank;
    auto bound_bits = [&](uint32_t k) -> uint32_t {  // 0: not in the pool
        const uint32_t m = s.meta[k], st = (m >> 1) & 3u;
        const float2 b = bw[k];
        const bool in = b.x > 0.0f && (st == T_EXPANDED || (st == T_LEAF && (m & 1u) && b.y > 0.0f));
        return in ? __float_as_uint(b.x) : 0u;
    };
    // fewer than R in the pool (early in a tree): every candidate may be committed
    if (tid == 0) s.band = 0;
    __syncthreads();
    uint32_t mine = 0;
    for (uint32_t k = tid; k < ntent; k += nt) mine += bound_bits(k) ? 1u : 0u;
    mine = wave_total(mine);
    if (lane == 0 && mine) atomicAdd(&s.band, mine);
    __syncthreads();
    if (s.band < R) return 0u;  // uniform
    __syncthreads();  // s.band is read before the rounds below set it
    uint32_t prefix = 0, mask = 0, above = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (uint32_t i = tid; i < 256u; i += nt) count[i] = 0;
        __syncthreads();
        for (uint32_t k = tid; k < ntent; k += nt) {
            const uint32_t v = bound_bits(k);
            if (v && (v & mask) == prefix) atomicAdd(&count[(v >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) {  // lane l: buckets 255 - 4 l down to 252 - 4 l
            uint32_t c = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) c += count[255u - 4u * lane - static_cast<uint32_t>(q)];
            const uint32_t incl = wave_incl_sum(c), before = incl - c;
            const unsigned long long hit = __ballot(above + incl >= R);
            if (!hit) {
                if (lane == 0) s.band = 256u;  // fewer than R in the pool
            } else if (lane == static_cast<uint32_t>(__builtin_ctzll(hit))) {
                uint32_t acc = above + before, b = 255u - 4u * lane;
                for (int q = 0; q < 4; ++q, --b) {
                    if (acc + count[b] >= R) break;
                    acc += count[b];
                }
                s.band = b;
                s.above = acc;
            }
        }
        __syncthreads();
        const uint32_t b = s.band;
        if (b == 256u) return 0u;  // uniform
        above = s.above;
        prefix |= b << shift;
        mask |= 255u << shift;
        __syncthreads();  // the counts are read before the next round clears them
    }
    return prefix;
}

template <uint32_t MAXL>
__device__ void advance(const GrowState &g, StepPlan &next, void *scratch) {
    AdvShared<MAXL> &s = *reinterpret_cast<AdvShared<MAXL> *>(scratch);
    GrowCtl *ctl = g.ctl;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, nt = blockDim.x;
    if (ctl->done) return;
    const uint32_t n0 = ctl->num_leaves, ntent = ctl->ntent, L = g.num_leaves;
    const uint32_t pending0 = ctl->pending, slot0 = ctl->next_slot, epoch0 = ctl->epoch;
    const uint32_t expansions0 = ctl->expansions, steps0 = ctl->steps;
    __syncthreads();  // every thread has read the control block before thread 0 updates it
    for (uint32_t k = tid; k < ntent; k += nt) {
        const TKey key = g.tk[k];
        s.gain[k] = key.gain;
        s.meta[k] = key_meta(key);
    }
    for (uint32_t id = tid; id < n0; id += nt) {
        s.leaf_t[id] = static_cast<uint16_t>(g.leaf_t[id]);
        s.pnode[id] = static_cast<int16_t>(g.tree.leaf_parent[id]);
        s.is_left[id] = g.leaf_left[id];
        s.touched[id] = 0;
    }
    if (tid == 0) {
        s.ncand = 0;
        s.nnan = 0;
    }
    __syncthreads();
    // the replay keys of the committed leaves for replay_lds and replay_reg (trees of more than 128 leaves), by the
    // whole block
    if (MAXL > LEAVES_SMALL || L > 128) {
        using Key = std::remove_cv_t<std::remove_reference_t<decltype(s.key[0])>>;
        for (uint32_t id = tid; id < MAXL; id += nt) {
            Key key = 0;
            if (id < n0) {
                const uint32_t t = s.leaf_t[id];
                const double gj = s.gain[t];
                const uint32_t m = s.meta[t];
                key = leaf_key<Key>(gj, m, id);
                if ((m & 1u) && gj != gj) atomicAdd(&s.nnan, 1u);
                if constexpr (MAXL > LEAVES_SMALL) s.leaf_m[id] = m;
            }
            s.key[id] = key;
        }
        if constexpr (MAXL <= LEAVES_SMALL) {  // replay_reg's records of the expanded speculative leaves
            for (uint32_t k = tid; k < ntent; k += nt) {
                const uint32_t m = s.meta[k];
                if (((m >> 1) & 3u) != T_EXPANDED) continue;
                const uint32_t kid = (m >> 3) - 1u;
                uint32_t c[2];
#pragma unroll
                for (uint32_t i = 0; i < 2; ++i) {
                    const double gc = s.gain[kid + i];
                    const uint32_t mc = s.meta[kid + i];
                    c[i] = (replay_key<11>(gc, mc, 0) & ~2047u) | ((mc & 1u) && gc != gc ? 1u : 0u);
                }
                s.crec[k] = make_uint2(c[0], c[1]);
            }
        }
        __syncthreads();
    }

    // -- the replay, one wave, with as few leaves per lane as the tree needs
    if (tid < 64) {
        if constexpr (MAXL <= LEAVES_SMALL) {
            if (L <= 64) replay<1>(s, n0, L);
            else if (L <= 128) replay<2>(s, n0, L);
            else if (L <= 256) replay_reg<4>(s, n0, L);
            else replay_reg<LEAVES_SMALL / 64>(s, n0, L);
        } else {
            if (L <= 1024) replay_lds<16>(s, n0, L);
            else replay_lds<MAXL / 64>(s, n0, L);
        }
    }
    __syncthreads();
    const uint32_t nc = s.ncommit, n = s.n;
    const bool done = s.done != 0;

    if (tid == 0) {
        ctl->num_leaves = n;
        ctl->pending = pending0 - nc;
        if (done) ctl->done = 1;
    }
    if (done) {
        apply_commits(g, s, n0, nc, n, 0, nt >> 6);
        return;
    }

    // -- speculation candidates: unexpanded leaves with a positive gain, the blocker aside, in the order best_leaf
    // would reach them: by bound (frontier_bounds), then gain, then lower leaf
    const uint32_t blocker = s.blocker;
    frontier_bounds<MAXL>(s, ntent, n);
    const uint32_t R = L - n;  // splits left, this step's blocker included
    // The pool holds the candidates, the blocker and the expanded leaves not yet committed (pending0 - nc). With
    // R >= that last count + jcap, fewer than R of them lie above the (jcap - 1)-th highest candidate's bound, so the
    // R-th highest bound cannot leave out any of the candidates a step takes: no selection is needed.
    const uint32_t cut = R >= pending0 - nc + g.jcap ? 0u : pool_threshold<MAXL>(s, ntent, R);
    if (tid == 0) s.neligible = 0;
    __syncthreads();
    const float2 *bw = reinterpret_cast<const float2 *>(s.gain);
    for (uint32_t k = tid; k < ntent; k += nt) {
        const uint32_t m = s.meta[k];
        const float2 b = bw[k];
        if ((m & 1u) && ((m >> 1) & 3u) == T_LEAF && b.y > 0.0f && b.x > 0.0f && k != blocker) {
            if (__float_as_uint(b.x) >= cut) atomicAdd(&s.neligible, 1u);
            const uint32_t at = atomicAdd(&s.ncand, 1u);
            s.cand[at] = static_cast<uint16_t>(k);
            // positive f32 bits order as the values: bound, then the top 19 bits of the gain below the sign, then
            // the lower leaf (13 bits: leaf ids are below 8192)
            s.ckey[at] = (static_cast<uint64_t>(__float_as_uint(b.x)) << 32) |
                         (static_cast<uint64_t>(__float_as_uint(b.y) >> 12) << 13) | (8191u - k);
            s.crank[at] = 0;
        }
    }
    __syncthreads();
    const uint32_t ncand = s.ncand;
    const uint32_t pending = pending0 - nc;
    // the candidates among the R leaves of highest bound (pool_threshold), at most jcap - 1; being the highest keys,
    // the ones the selection below takes are exactly those
    uint32_t spec = s.neligible;
    if (spec > g.jcap - 1) spec = g.jcap - 1;
    // room for this step and every later blocker (each commits, so at most R of them in all)
    const uint32_t free_t = g.tcap - ntent, free_s = g.nslots - slot0;
    const uint32_t room_t = free_t >= 2 * R ? (free_t - 2 * R) / 2 : 0u, room_s = free_s >= R ? free_s - R : 0u;
    if (spec > room_t) spec = room_t;
    if (spec > room_s) spec = room_s;
    if (spec > ncand) spec = ncand;
    // The spec highest keys; the blocker is job 0. Which leaves are expanded early changes no result (every
    // expansion is the one its leaf gets when the replay reaches it), only the work done ahead. Up to 512 candidates,
    // each one's rank (keys above its own) is summed over `nsl` slices of the others, one thread each; beyond that
    // (trees of thousands of leaves), a radix selection finds the spec-th key in linear passes.
    if (spec <= SPEC_FEW) {
        if (tid < 64) top_few(s, ncand, spec);
    } else if (ncand <= 512u) {
        const uint32_t nsl = ncand && ncand < nt ? nt / ncand : 1u;
        for (uint32_t w = tid; w < ncand * nsl; w += nt) {
            const uint32_t i = w % ncand, sl = w / ncand;
            const uint64_t ki = s.ckey[i];
            uint32_t rank = 0;
#pragma unroll 8
            for (uint32_t j = sl; j < ncand; j += nsl) rank += s.ckey[j] > ki ? 1u : 0u;
            atomicAdd(&s.crank[i], rank);
        }
        __syncthreads();
        for (uint32_t i = tid; i < ncand; i += nt)
            if (s.crank[i] < spec) s.job_t[1 + s.crank[i]] = s.cand[i];
    } else {
        select_top<MAXL>(s, ncand, spec);
    }
    if (tid == 0) {
        s.job_t[0] = static_cast<uint16_t>(blocker);
        s.njobs = 1 + spec;
    }
    __syncthreads();
    const uint32_t njobs = s.njobs;
    if (free_t < 2 || free_s < 1) {  // no room even for the blocker: the sizes above make this unreachable
        if (tid == 0) {
            ctl->error = 4;
            ctl->done = 1;
        }
        apply_commits(g, s, n0, nc, n, 0, nt >> 6);
        return;
    }

    // -- the jobs (learner.rs:249-290), one lane each; then prefix sums over the jobs on the same wave. The other
    // waves meanwhile apply the commits to the tree (nothing the plan reads).
    if (tid >= 64) apply_commits(g, s, n0, nc, n, 1, (nt >> 6) - 1);
    if (tid < 64) {
        const bool on = lane < njobs;
        JobPlan J = {};
        uint32_t hist = 0, ntiles = 0;
        float cost = 0.0f;
        if (on) {
            const uint32_t tt = s.job_t[lane];
            const TLeaf &l = g.tl[tt];
            const SplitOut &info = l.best;
            J.t = tt;
            J.begin = l.begin;
            J.count = l.count;
            J.col = info.col;
            J.wide = g.feats[info.feature].wide;
#pragma unroll
            for (uint32_t w = 0; w < 8; ++w) J.left_bins[w] = left_bins_word(info, w, J.wide);
            J.built_side = info.left_count <= info.right_count ? 0u : 1u;
            hist = (l.slot >= 0 && depth_allows(g, l.depth + 1)) ? 1u : 0u;
            J.hist = hist;
            J.parent_slot = l.slot;
            J.src_buf = l.buf;
            J.src_rev = l.rev;
            ntiles = (l.count + STEP_TILE - 1) / STEP_TILE;
            J.ntiles = ntiles;
            // the job's k_step_rows work in tiles: every tile partitions, its rows' split bins costing more the sparser
            // the leaf's rows lie (a line a row once they are sparser than one in 128: sparse_weight at most), and the
            // built child's share of its rows is histogrammed besides (hist_weight a tile of built rows)
            const double lc = static_cast<double>(info.left_count), rc = static_cast<double>(info.right_count);
            const double built = hist && lc + rc > 0.0 ? (lc <= rc ? lc : rc) / (lc + rc) : 0.0;
            const double spread = static_cast<double>(g.tl[0].count) / (128.0 * static_cast<double>(l.count ? l.count : 1u));
            cost = static_cast<float>(ntiles) * (1.0f + g.sparse_weight * static_cast<float>(spread < 1.0 ? spread : 1.0) +
                                                 g.hist_weight * static_cast<float>(built));
            J.parent_count = l.cnt;
            J.child_ug[0] = info.left_grad;
            J.child_uh[0] = info.left_hess;
            J.child_ug[1] = info.right_grad;
            J.child_uh[1] = info.right_hess;
            J.kid = static_cast<int32_t>(ntent + 2 * lane);
        }
        // exclusive prefixes over lanes 0..njobs-1 (one wave)
        const uint32_t hist_before = wave_excl_sum(hist);
        const uint32_t tiles_before = wave_excl_sum(ntiles);
        const uint32_t total_tiles = wave_total(ntiles);
        const float total_cost = wave_total_f32(cost);
        uint32_t groups = 0;
        if (on) {  // workgroups in proportion to the jobs' work (a job's tiles go to its workgroups by ticket), so that
            // no job's workgroups run long; the rounding up in each job costs at most one workgroup a job, so with
            // target - njobs for the shares the step fits in one round of workgroups (one per compute unit). At most
            // tile_cap tiles a workgroup (its i32 sums), and no more workgroups than tiles.
            const uint32_t share = g.target_groups > njobs ? g.target_groups - njobs : 1u;
            if (total_tiles <= g.target_groups) {
                groups = ntiles;
            } else {
                const float per_cost = total_cost / static_cast<float>(share);
                groups = static_cast<uint32_t>(__builtin_ceilf(cost / per_cost));
                const uint32_t least = (ntiles + g.tile_cap - 1) / g.tile_cap;
                groups = groups < least ? least : groups;
                groups = groups > ntiles ? ntiles : groups;
            }
            if (groups == 0) groups = 1;
        }
        const uint32_t groups_before = wave_excl_sum(groups);
        const uint32_t total_groups = wave_total(groups);
        uint32_t red = 0, scan = 0;
        if (on) {
            J.tile_base = tiles_before;
            J.groups = groups;
            J.group_base = groups_before;
            J.packed = (ntiles <= groups && g.flush_rows >= STEP_TILE) ? 1u : 0u;
            J.ways = reduce_ways(groups);
            red = hist ? g.ncg * J.ways : 0u;
            scan = hist ? g.nsg : 0u;
            J.red_items = red;
            J.scan_items = scan;
            J.built_slot = hist ? static_cast<int32_t>(slot0 + hist_before) : -1;
        }
        const uint32_t red_before = wave_excl_sum(red), scan_before = wave_excl_sum(scan);
        const uint32_t total_red = wave_total(red), total_scan = wave_total(scan);
        const uint32_t nhist = wave_total(hist);
        if (on) {
            J.red_base = red_before;
            J.scan_base = scan_before;
            next.group_base[lane] = J.group_base;
            next.red_base[lane] = red_before;
            next.scan_base[lane] = scan_before;
            J.ticket = 0;
            J.left = 0;
            next.jobs[lane] = J;
            g.tl[J.t].state = T_PLANNED;
            g.tl[J.t].kid = J.kid;
            g.tk[J.t].state = T_PLANNED;
            g.tk[J.t].kid = J.kid;
        }
        if (lane == 0) {
            next.njobs = njobs;
            next.total_groups = total_groups;
            next.total_red = total_red;
            next.total_scan = total_scan;
            next.epoch = epoch0 + 1;
            ctl->epoch = epoch0 + 1;
            ctl->ntent = ntent + 2 * njobs;
            ctl->next_slot = slot0 + nhist;
            ctl->pending = pending + njobs;
            ctl->expansions = expansions0 + njobs;
            ctl->steps = steps0 + 1;
        }
    }
}

// After a grown tree's steps: when the tree is complete with at least one split, its nodes for k_tree_leaves and
// k_add_tree (as the host builds them from the tree it reads back: the split's bins, the column of its feature,
// the children), its leaf sums zeroed, and *gate = its leaves; *gate = 0 otherwise (an unfinished tree or one
// that never split: the gated kernels after it do nothing). Every node is checked as the host checks an uploaded
// tree (a known feature; an internal child after its parent, a leaf child among the leaves), so the walks over it
// end; a malformed tree flags ctl->error = 6 and closes the gate. *gate_out: the gate, for the host. A nonzero
// *veto (when given: the iteration's gradients are to be made again) closes the gate too. One block.
__global__ void k_tree_nodes(GrowState g, DevNode *nodes, unsigned long long *sums, uint32_t *gate, double *gate_out,
                             const uint32_t *veto) {
    __shared__ uint32_t bad;
    GrowCtl *ctl = g.ctl;
    const uint32_t n = ctl->done && !ctl->error && !(veto && *veto) ? ctl->num_leaves : 0u;
    const uint32_t nl = n > 1u && n <= GROW_MAX_LEAVES ? n : 0u, nn = nl ? nl - 1u : 0u;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    for (uint32_t k = threadIdx.x; k < nn; k += blockDim.x) {
        DevNode d;
#pragma unroll
        for (int w = 0; w < 8; ++w) d.left_bins[w] = g.tree.left_bins[static_cast<size_t>(k) * 8 + w];
        const int32_t f = g.tree.split_feature[k];
        d.feature = f >= 0 && static_cast<uint32_t>(f) < g.nf ? g.feats[f].col : 0u;
        d.left = g.tree.left_child[k];
        d.right = g.tree.right_child[k];
        d.wide = f >= 0 && static_cast<uint32_t>(f) < g.nf ? g.feats[f].wide : 0u;
        nodes[k] = d;
        bool ok = f >= 0 && static_cast<uint32_t>(f) < g.nf;
        for (const int32_t c : {d.left, d.right})
            ok = ok && (c >= 0 ? static_cast<uint32_t>(c) > k && static_cast<uint32_t>(c) < nn : static_cast<uint32_t>(~c) < nl);
        if (!ok) atomicOr(&bad, 1u);
    }
    for (uint32_t i = threadIdx.x; i < 2u * nl; i += blockDim.x) sums[i] = 0ull;
    __syncthreads();
    if (threadIdx.x == 0) {
        if (bad) ctl->error = 6;
        *gate = bad ? 0u : nl;
        *gate_out = static_cast<double>(bad ? 0u : nl);
    }
}

// The root's best split (learner.rs:157-163), then the first step's plan. One block of 512 threads; MAXL: the
// largest tree it takes (LEAVES_SMALL or GROW_MAX_LEAVES).
template <uint32_t MAXL>
__global__ __launch_bounds__(512) void k_root_select(GrowState g) {
    __shared__ SplitOut o;
    __shared__ __align__(16) uint8_t scratch[sizeof(AdvShared<MAXL>)];
    ScanJob job = g.jobs[0];
    select_split(job, job.count, g.nf, g.cfg, grow_sg(g), grow_sh(g), &o, g.splittable);
    if (threadIdx.x == 0) {
        g.tl[0].best = o;
        g.tl[0].has_best = o.found ? 1u : 0u;
        g.tk[0].gain = o.gain;
        g.tk[0].has = o.found ? 1u : 0u;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __threadfence();
    advance<MAXL>(g, g.plans[0], scratch);
}

// ---------------------------------------------------------------------------------------------------------
// A split step in two kernels: every job of the step's plan (learner.rs:249-352 for each leaf it expands).
//
// k_step_rows: the stable partition of each job's rows by its BinSplit (cpu.rs:556-599) in one pass, fused with
// its built child's histogram. A job's workgroups take its tiles of STEP_TILE rows in order; a tile's left
// count is published at once, its offset comes from a look-back over the job's earlier tiles (no second pass
// over the rows), its rows are scattered, then its rows of the built child (kept in LDS) are histogrammed as
// k_hist does. Left rows are written first-first from the range's start, right rows last-first from its end, so
// both children are stable; a leaf stored last-first is read back to front by the step that expands it and by
// k_consolidate. Launches for a second or later slab only histogram.
//
// Then, one launch each: k_step_reduce adds each job's partials (work items: job, column group, bin range), writes
// the built child's histogram and forms the sibling by subtraction (learner.rs:356-371); k_step_scan and
// k_step_cat scan every (job, feature, child); k_step_select selects both children's splits of each job
// (job_select), and its last block to finish runs advance. That hand-off is a counter the last arriving block
// resets; no block ever waits for another.
// ---------------------------------------------------------------------------------------------------------

// A launch takes one slab, or (histogram only) several slabs of one kernel, k1 workgroups each: slab s of the
// launch is the first one's buffers moved by s strides (its rows by bins_stride bytes, its partials by k1
// partials, its formats by k1 entries, its column bins by W * PACK entries).
struct StepArgs {
    const uint8_t *bins;         // the first slab's rows: row r at bins + r * row bytes
    uint64_t bins_stride;
    int32_t *partial;            // its partials, step_partial_stride(W) pairs apart, one per workgroup
    uint32_t *fmt;               // per workgroup: its partial is packed (1) or {g, h} pairs (0)
    const uint32_t *col_bins;    // per slab column: its feature's bins (0 for padding)
    const uint32_t *pos_word;    // a dense slab: per row byte, its LDS word at bin 0 (256 * DP entries a slab)
    uint32_t dw_row;             // a dense slab: dwords per row
    uint32_t k1;                 // workgroups a slab
    const int32_t *gh;           // packed quantized gradients per row
    const uint8_t *colbase;      // column-major bins [feature][rows]
    uint32_t col16;              // two bytes per column-major bin
    uint64_t rows;
    uint32_t *buf0, *buf1;       // the partition buffers
    unsigned long long *status;  // per-tile status words
    StepPlan *plan;              // this step's plan
    GrowCtl *ctl;
    uint32_t flush_rows;
    uint32_t partition;          // 1: this launch partitions (the first slab's alone); 0: histogram only
    uint32_t tile_cap;           // tiles a workgroup takes at most (its i32 sums of the quantized units)
    uint8_t *codes0, *codes1;    // each row's one-byte gradient code beside its id in buf0 / buf1 (packed_code), or
                                 // null: the histograms gather the packed words
};

__device__ __forceinline__ unsigned long long status_word(uint32_t epoch, uint32_t flag, uint32_t value) {
    return (static_cast<unsigned long long>(((epoch & 0x3fffffffu) << 2) | flag) << 32) | value;
}

// Lefts in the tiles before `t`: wave-wide over up to 64 earlier tiles at a time, nearest first, summing
// aggregates until an inclusive prefix. Tile 0 always publishes an inclusive one, and every earlier tile was
// handed to a running block that publishes its aggregate before any wait, so the polling ends; a step that
// still sees no status after LOOKBACK_SPINS polls flags an error instead of waiting on.
__device__ uint32_t lookback(const unsigned long long *status, uint32_t t, uint32_t epoch, GrowCtl *ctl) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t want = epoch & 0x3fffffffu;
    uint32_t prefix = 0, spins = 0;
    int64_t hi = static_cast<int64_t>(t) - 1;
    while (hi >= 0) {
        const int64_t idx = hi - static_cast<int64_t>(lane);
        unsigned long long w = 0;
        if (idx >= 0) w = __hip_atomic_load(status + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t tag = static_cast<uint32_t>(w >> 32);
        const bool ready = idx >= 0 && (tag >> 2) == want && (tag & 3u) != 0u;
        const unsigned long long waiting = __ballot(idx >= 0 && !ready);
        const unsigned long long incl = __ballot(ready && (tag & 3u) == ST_INCL);
        const uint32_t first_incl = incl ? static_cast<uint32_t>(__builtin_ctzll(incl)) : 64u;
        const uint32_t first_wait = waiting ? static_cast<uint32_t>(__builtin_ctzll(waiting)) : 64u;
        if (first_wait < first_incl) {
            if (++spins > LOOKBACK_SPINS) {
                if (lane == 0) ctl->error = 3;
                return prefix;
            }
            __builtin_amdgcn_s_sleep(2);
            continue;
        }
        const uint32_t take = first_incl < 64u ? first_incl + 1u : 64u;
        uint32_t v = (lane < take && idx >= 0) ? static_cast<uint32_t>(w) : 0u;
        for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
        prefix += v;
        if (first_incl < 64u) break;
        hi -= 64;
    }
    return prefix;
}

// Moves the packed 16/16 LDS words (Q32: the separate g and h counters) into a workgroup's {g, h} pair partial
// (stored, or added to what an earlier flush stored) and zeroes them. Slot tid + 1024 j is bin (tid + 1024 j) / W
// of column tid % W; bins past the column's feature are not stored. Block-wide.
template <int W, bool Q32 = false>
__device__ __forceinline__ void flush_pairs(int32_t *lds, int2 *pairs, uint32_t col_bins, bool add) {
    constexpr int SLOTS = 256 * W / 1024;
    const uint32_t tid = threadIdx.x;
    __syncthreads();
#pragma unroll 8
    for (int j = 0; j < SLOTS; ++j) {
        const uint32_t slot = tid + j * 1024;
        const int32_t v = lds[slot];
        lds[slot] = 0;
        int32_t gq, hq;
        if constexpr (Q32) {
            gq = v;
            hq = lds[256 * W + slot];
            lds[256 * W + slot] = 0;
        } else {
            gq = packed_g(v);
            hq = packed_h(v, gq);
        }
        if (slot / W < col_bins) {
            int2 o = add ? pairs[slot] : make_int2(0, 0);
            o.x += gq;
            o.y += hq;
            pairs[slot] = o;
        }
    }
    __syncthreads();
}

// A job of the step as one workgroup of k_step_rows sees it.
struct StepView {
    JobPlan *job;
    unsigned long long *status;  // the job's tile status words
    uint32_t begin, count, ntiles, groups;
    const uint32_t *src;
    uint32_t *dst;
    bool rev, hist, partition;
    const uint8_t *col;
    uint32_t col16;       // column-major bins are two bytes
    uint32_t wide;        // the split is a wide feature's numerical rule
    uint32_t built_left;  // 1: the left child is histogrammed
    uint32_t epoch;
    const uint8_t *csrc;  // the rows' gradient codes beside src, and beside dst (CODES)
    uint8_t *cdst;
};

struct StepShared {
    uint32_t list[STEP_TILE];  // the tile's rows of the built child
    uint8_t codes[STEP_TILE];  // and their gradient codes (CODES)
    uint32_t wl[TILE_RPT][16];  // left counts per (sub-tile, wave)
    uint32_t left_bins[8];     // the split's bins that go left
    uint32_t tile, tile2, prefix;
};

// One partition tile in parts. tile_rows and tile_bins read its rows in the leaf's order (TILE_RPT per thread:
// positions tid, 1024 + tid, ...) and their split-feature bins, so that a workgroup can load its next tile while
// it works on this one; tile_front ranks the lefts, publishes the tile's left count and lists its rows of the built
// child in sh.list, in order; tile_lookback (wave 0) takes the tile's offset from the look-back; tile_scatter
// writes its rows, left first-first and right last-first. Between the last two the other waves histogram the
// listed rows.
struct TileRows {
    uint32_t row[TILE_RPT], bin[TILE_RPT];
    uint32_t codes;  // CODES: row j's gradient code in byte j
};

template <bool CODES>
__device__ __forceinline__ void tile_rows(const StepView &v, uint32_t t, TileRows &r) {
    const uint32_t t0 = t * STEP_TILE;
    static_assert(TILE_RPT <= 4, "a tile's codes fit one word a thread");
    if constexpr (CODES) r.codes = 0;
#pragma unroll
    for (int j = 0; j < TILE_RPT; ++j) {
        const uint32_t i = t0 + j * 1024 + threadIdx.x;
        const uint32_t ic = i < v.count ? i : v.count - 1;
        const uint32_t at = v.rev ? v.begin + v.count - 1 - ic : v.begin + ic;
        r.row[j] = v.src[at];
        if constexpr (CODES) r.codes |= static_cast<uint32_t>(v.csrc[at]) << (8 * j);
    }
}

__device__ __forceinline__ void tile_bins(const StepView &v, TileRows &r) {
#pragma unroll
    for (int j = 0; j < TILE_RPT; ++j) r.bin[j] = col_bin(v.col, v.col16, r.row[j]);
}

struct TileState {
    uint32_t row[TILE_RPT], lrank[TILE_RPT];  // lrank: lefts before the row in the tile
    uint32_t codes;                           // CODES: row j's gradient code in byte j
    bool ok[TILE_RPT], left[TILE_RPT];
    uint32_t tile_left;
};

// Returns the rows listed. Block-wide; the list is complete on return.
template <bool CODES>
__device__ __forceinline__ uint32_t tile_front(const StepView &v, uint32_t t, const TileRows &r, TileState &st,
                                               StepShared &sh) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint64_t below_mask = (1ull << lane) - 1ull;
    const uint32_t t0 = t * STEP_TILE;
    const uint32_t valid = v.count - t0 < STEP_TILE ? v.count - t0 : STEP_TILE;
    if constexpr (CODES) st.codes = r.codes;
#pragma unroll
    for (int j = 0; j < TILE_RPT; ++j) {
        st.ok[j] = t0 + j * 1024 + tid < v.count;
        st.row[j] = r.row[j];
        st.left[j] = st.ok[j] && rule_left(sh.left_bins, v.wide, r.bin[j]);
    }
    uint32_t below[TILE_RPT];
#pragma unroll
    for (int j = 0; j < TILE_RPT; ++j) {
        unsigned long long m = __ballot(st.left[j]);
        below[j] = static_cast<uint32_t>(__popcll(m & below_mask));
        if (lane == 0) sh.wl[j][wave] = static_cast<uint32_t>(__popcll(m));
    }
    __syncthreads();
    // lefts before each row of the tile (rows in order: sub-tile, wave, lane)
    uint32_t sub[TILE_RPT], before[TILE_RPT];
#pragma unroll
    for (int j = 0; j < TILE_RPT; ++j) sub[j] = before[j] = 0;
    for (uint32_t w = 0; w < 16; ++w) {
#pragma unroll
        for (int j = 0; j < TILE_RPT; ++j) {
            const uint32_t c = sh.wl[j][w];
            sub[j] += c;
            before[j] += w < wave ? c : 0u;
        }
    }
    st.tile_left = 0;
#pragma unroll
    for (int j = 0; j < TILE_RPT; ++j) {
        st.lrank[j] = st.tile_left + before[j] + below[j];
        st.tile_left += sub[j];
    }
    if (v.partition && tid == 0)
        __hip_atomic_store(v.status + t, status_word(v.epoch, t == 0 ? ST_INCL : ST_AGG, st.tile_left), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    if (v.hist) {  // the tile's rows of the built child, in order
#pragma unroll
        for (int j = 0; j < TILE_RPT; ++j) {
            uint32_t pos = j * 1024 + tid;
            if (st.ok[j] && (st.left[j] ? 1u : 0u) == v.built_left) {
                const uint32_t at = v.built_left ? st.lrank[j] : pos - st.lrank[j];
                sh.list[at] = st.row[j];
                if constexpr (CODES) sh.codes[at] = static_cast<uint8_t>(st.codes >> (8 * j));
            }
        }
    }
    __syncthreads();  // the list is complete
    return v.built_left ? st.tile_left : valid - st.tile_left;
}

// The tile's offset into sh.prefix, published as its inclusive count. Wave 0 of a partition launch.
__device__ __forceinline__ void tile_lookback(const StepView &v, const StepArgs &a, uint32_t t, const TileState &st,
                                              StepShared &sh) {
    const uint32_t prefix = t == 0 ? 0u : lookback(v.status, t, v.epoch, a.ctl);
    if ((threadIdx.x & 63u) == 0) {
        if (t > 0)
            __hip_atomic_store(v.status + t, status_word(v.epoch, ST_INCL, prefix + st.tile_left), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        sh.prefix = prefix;
        if (t == v.ntiles - 1) v.job->left = prefix + st.tile_left;
    }
}

// The tile's rows written from the offset in sh.prefix (after a barrier that follows tile_lookback).
template <bool CODES>
__device__ __forceinline__ void tile_scatter(const StepView &v, uint32_t t, const TileState &st, const StepShared &sh) {
    const uint32_t tid = threadIdx.x;
    const uint32_t lp = sh.prefix, rp = t * STEP_TILE - lp;  // lefts and rights before the tile
#pragma unroll
    for (int j = 0; j < TILE_RPT; ++j) {
        if (!st.ok[j]) continue;
        uint32_t at;
        if (st.left[j]) {
            const uint32_t k = lp + st.lrank[j];
            if (k >= v.count) continue;
            at = v.begin + k;
        } else {
            const uint32_t k = rp + (j * 1024 + tid - st.lrank[j]);
            if (k >= v.count) continue;
            at = v.begin + v.count - 1 - k;
        }
        v.dst[at] = st.row[j];
        if constexpr (CODES) v.cdst[at] = static_cast<uint8_t>(st.codes >> (8 * j));
    }
}

// The histogram of rows list[c0, c1) into the packed LDS words: a wave covers RPW = 64 / (W/4) rows per step, a
// lane one dword (4 columns) of a row, with the conflict-free byte rotation of k_hist. Loads are branch-free. NW
// waves take part; `wave` is this one's index among them.
template <int W, bool WIDE, int PACK, bool Q32, int UNROLL, int NW = 16, bool CODES = false>
__device__ __forceinline__ void hist_list(int32_t *lds, const uint32_t *list, uint32_t c0, uint32_t c1, const int32_t *gh,
                                          const uint32_t *bins32, uint32_t wave = threadIdx.x >> 6,
                                          const uint8_t *codes = nullptr) {
    constexpr int DW = WIDE ? W / 8 : W * PACK / 4;
    constexpr int RPW = WAVE / DW;
    constexpr uint32_t STEP = NW * RPW * UNROLL;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t d = lane % DW, rsub = lane / DW;
    const uint32_t rot = (lane & 31u) >> 3;
    uint32_t xs[4], cols[4];
    row_bin_lanes<W, PACK>(d, rot, xs, cols);
    const uint32_t last = c1 - 1;
    for (uint32_t base = c0 + wave * RPW * UNROLL; base < c1; base += STEP) {
        uint32_t r[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) r[u] = list[min(base + u * RPW + rsub, last)];
        uint32_t dw[UNROLL];
        int32_t gq[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            if constexpr (CODES) gq[u] = code_word(codes[min(base + u * RPW + rsub, last)]);
            else gq[u] = gh[r[u]];
            dw[u] = bins32[static_cast<size_t>(r[u]) * DW + d];
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            int32_t gv, hv;
            row_units<Q32>(gq[u], base + u * RPW + rsub < c1, gv, hv);
            if constexpr (WIDE) add_row_bins_wide<W, Q32>(lds, dw[u], gv, hv, d);
            else add_row_bins<W, PACK, Q32>(lds, dw[u], gv, hv, xs, cols);
        }
    }
}

// A workgroup's packed LDS words (every row added, none flushed) stored as its partial: int4 q * W + c holds bin
// 4q + c % 4 of columns (c & ~3) .. (c & ~3) + 3. Task k takes column c = k % W and bins 4q..4q+3 (q = k / W),
// reads LDS across the wave without bank conflicts, and a butterfly transpose in each quad of lanes (the group's 4
// columns) leaves lane c % 4 with bin 4q + c % 4 of all four columns: a wave stores 1 KiB contiguously. The LDS
// words must be complete (after a barrier). Block-wide, 1024 threads.
template <int W>
__device__ __forceinline__ void store_packed_partial(const int32_t *lds, int32_t *partial) {
    constexpr int SLOTS = 256 * W / 1024;
    int4 *out = reinterpret_cast<int4 *>(partial);
    const uint32_t tid = threadIdx.x, c4 = tid & 3u;
#pragma unroll
    for (int it = 0; it < SLOTS / 4; ++it) {
        const uint32_t k = tid + 1024u * it, c = k % W, q = k / W;
        int32_t v0 = lds[(4 * q + 0) * W + c], v1 = lds[(4 * q + 1) * W + c];
        int32_t v2 = lds[(4 * q + 2) * W + c], v3 = lds[(4 * q + 3) * W + c];
        // at level b a lane keeps the elements whose index bit b matches its own and swaps the other two with
        // lane c4 ^ b; every choice is one select on a lane bit
        {
            const bool hi = (c4 & 1u) != 0;
            const int32_t t0 = __builtin_amdgcn_update_dpp(0, hi ? v0 : v1, 0xB1, 0xf, 0xf, false);
            const int32_t t1 = __builtin_amdgcn_update_dpp(0, hi ? v2 : v3, 0xB1, 0xf, 0xf, false);
            const int32_t n0 = hi ? t0 : v0, n1 = hi ? v1 : t0, n2 = hi ? t1 : v2, n3 = hi ? v3 : t1;
            v0 = n0;
            v1 = n1;
            v2 = n2;
            v3 = n3;
        }
        {
            const bool hi = (c4 & 2u) != 0;
            const int32_t t0 = __builtin_amdgcn_update_dpp(0, hi ? v0 : v2, 0x4E, 0xf, 0xf, false);
            const int32_t t1 = __builtin_amdgcn_update_dpp(0, hi ? v1 : v3, 0x4E, 0xf, 0xf, false);
            const int32_t n0 = hi ? t0 : v0, n1 = hi ? t1 : v1, n2 = hi ? v2 : t0, n3 = hi ? v3 : t1;
            v0 = n0;
            v1 = n1;
            v2 = n2;
            v3 = n3;
        }
        out[q * W + c] = make_int4(v0, v1, v2, v3);  // column (c & ~3) + j at bin 4q + c4
    }
}

// hist_list for a 128-column byte slab with 8 columns a lane: a wave covers 4 rows a step, lane l the dword pair
// l % 16 of row l / 16, so a row is one 128-byte line read by 16 lanes and a wave has 4 * UNROLL rows in flight for
// the registers that 2 * UNROLL rows take at a dword a lane. Each lane rotates its pair right by `rot` bytes once a
// row, so that its k-th add takes byte (k + rot) % 8 (column 8d + (k + rot) % 8). The LDS serves an instruction a
// half-wave (32 lanes, two rows) at a time; with rot = d / 4 + 4 * (row % 2) the 8 lanes of a half-wave whose
// columns share a bank group (d % 4 alike) take 8 different bytes, so no two of its lanes meet in a bank.
template <int UNROLL, int NW = 16, bool CODES = false>
__device__ __forceinline__ void hist_list_pairs(int32_t *lds, const uint32_t *list, uint32_t c0, uint32_t c1,
                                                const int32_t *gh, const uint32_t *bins32, uint32_t wave,
                                                const uint8_t *codes = nullptr) {
    constexpr uint32_t W = 128, RPW = 4;
    constexpr uint32_t STEP = NW * RPW * UNROLL;
    const uint32_t lane = threadIdx.x & 63u, d = lane & 15u, rsub = lane >> 4;
    const uint32_t rot = ((d >> 2) + 4u * (rsub & 1u)) & 7u;
    const bool swap = rot >= 4u;
    const uint32_t sh = 8u * (rot & 3u);
    uint32_t cols[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) cols[k] = 8u * d + ((static_cast<uint32_t>(k) + rot) & 7u);
    const uint2 *rows2 = reinterpret_cast<const uint2 *>(bins32);
    const uint32_t last = c1 - 1;
    for (uint32_t base = c0 + wave * RPW * UNROLL; base < c1; base += STEP) {
        uint32_t r[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) r[u] = list[min(base + u * RPW + rsub, last)];
        uint2 v[UNROLL];
        int32_t gq[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            if constexpr (CODES) gq[u] = code_word(codes[min(base + u * RPW + rsub, last)]);
            else gq[u] = gh[r[u]];
            v[u] = rows2[static_cast<size_t>(r[u]) * (W / 8) + d];
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int32_t gv = base + u * RPW + rsub < c1 ? gq[u] : 0;
            const uint32_t a = swap ? v[u].y : v[u].x, b = swap ? v[u].x : v[u].y;  // the pair rotated by 4 bytes
            const uint32_t lo = __builtin_amdgcn_alignbit(b, a, sh), hi = __builtin_amdgcn_alignbit(a, b, sh);
#pragma unroll
            for (int k = 0; k < 4; ++k) atomicAdd(&lds[__builtin_amdgcn_ubfe(lo, 8u * k, 8u) * W + cols[k]], gv);
#pragma unroll
            for (int k = 0; k < 4; ++k) atomicAdd(&lds[__builtin_amdgcn_ubfe(hi, 8u * k, 8u) * W + cols[4 + k]], gv);
        }
    }
}

// A split step's histogram of list[c0 .. c1): hist_list, or hist_list_dense for a dense slab (DP passes).
template <int W, bool WIDE, int PACK, bool Q32, int DP, int UNROLL, int NW = 16, bool CODES = false>
__device__ __forceinline__ void step_hist(int32_t *lds, const uint32_t *list, uint32_t c0, uint32_t c1, const int32_t *gh,
                                          const uint32_t *bins32, uint32_t dw_row, const uint32_t (&xs)[4],
                                          const uint32_t (&dcols)[DP ? DP : 1][4], uint32_t wave = threadIdx.x >> 6,
                                          const uint8_t *codes = nullptr) {
    if constexpr (DP > 0)
        hist_list_dense<W, DP, DP <= 4 ? 2 : 1, NW, CODES>(lds, list, c0, c1, gh, bins32, dw_row, xs, dcols, wave, codes);
    else if constexpr (W == 128 && !WIDE && PACK == 1 && !Q32)
        hist_list_pairs<UNROLL * 3 / 4, NW, CODES>(lds, list, c0, c1, gh, bins32, wave, codes);
    else hist_list<W, WIDE, PACK, Q32, UNROLL, NW, CODES>(lds, list, c0, c1, gh, bins32, wave, codes);
}

// The one-byte gradient codes of a tree's root rows, beside their ids: codes[i] = packed_code(gh[part[i]]) for i in
// [begin, begin + count). The split steps then move each code with its row. Four rows a thread, their loads issued
// together (one row a thread waited on two dependent loads a row).
__global__ void k_gh_codes(const uint32_t *__restrict__ part, const int32_t *__restrict__ gh, uint32_t begin,
                           uint32_t count, uint8_t *__restrict__ codes) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < count; i += 4u * stride) {
        uint32_t r[4];
        int32_t w[4];
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) r[k] = i + k * stride < count ? part[begin + i + k * stride] : 0u;
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) w[k] = i + k * stride < count ? gh[r[k]] : 0;
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k)
            if (i + k * stride < count) codes[begin + i + k * stride] = packed_code(w[k]);
    }
}

// The LDS words of a k_step_rows instance: the histogram (twice for separate counters) and a dense slab's spare row.
template <int W, bool Q32, int DP>
constexpr int step_lds_words() { return (Q32 ? 2 : 1) * 256 * W + (DP ? W : 0); }

// k_step_rows' work, with the built rows' gradients read from their carried codes (CODES) or gathered.
template <int W, bool WIDE, int PACK, bool Q32, int DP, bool CODES>
__device__ __forceinline__ void step_rows_body(const StepArgs &a, int32_t *lds, StepShared &sh) {
    static_assert(PACK == 1 || (!WIDE && W * PACK <= 256), "a packed row is at most 64 dwords");
    static_assert(!Q32 || W <= 64, "separate g and h counters take twice the LDS");
    static_assert(DP == 0 || (W == 128 && !WIDE && PACK == 1 && !Q32), "a dense slab has 128 byte columns");
    static_assert(!(CODES && Q32), "codes hold small units only");
    constexpr int DW = WIDE ? W / 8 : W * PACK / 4;
    constexpr int RPW = WAVE / DW;
    // rows per lane in multi-tile workgroups (16 at W = 32 with packed columns spills)
    constexpr int UNROLL = (W == 128 || (W == 32 && PACK > 1)) ? 8 : (64 / RPW < 16 ? 64 / RPW : 16);
    constexpr int SLOTS = 256 * W / 1024;
    constexpr int LDS_WORDS = step_lds_words<W, Q32, DP>();

    // a launch of histogram-only slabs takes k1 workgroups a slab: wg is the workgroup within its slab
    const uint32_t sl = blockIdx.x / a.k1, wg = blockIdx.x - sl * a.k1;
    struct {
        const uint8_t *bins;
        int32_t *partial;
        uint32_t *fmt;
        const uint32_t *col_bins;
        const uint32_t *pos_word;
    } R = {a.bins + sl * a.bins_stride, a.partial + static_cast<size_t>(sl) * a.k1 * 2 * step_partial_stride(W),
           a.fmt + sl * a.k1, a.col_bins + sl * (W * PACK), a.pos_word + sl * 256u * (DP ? DP : 1)};
    StepPlan &P = *a.plan;  // empty once the tree is done (k_step_select)
    if (wg >= P.total_groups) return;
    const uint32_t j = job_of(P.group_base, P.njobs, wg);
    JobPlan &J = P.jobs[j];
    StepView v;
    v.job = &J;
    v.hist = J.hist != 0;
    v.partition = a.partition != 0;
    if (!v.hist && !v.partition) return;
    v.status = a.status + J.tile_base;
    v.begin = J.begin;
    v.count = J.count;
    v.ntiles = J.ntiles;
    v.groups = J.groups;
    const uint32_t gi = wg - J.group_base;  // the workgroup within its job
    const bool packed = J.packed != 0;  // then one tile per workgroup
    v.src = J.src_buf ? a.buf1 : a.buf0;
    v.dst = J.src_buf ? a.buf0 : a.buf1;
    v.rev = J.src_rev != 0;
    v.col16 = a.col16;
    v.wide = J.wide;
    v.col = a.colbase + static_cast<size_t>(J.col) * a.rows * (a.col16 ? 2u : 1u);
    v.built_left = J.built_side == 0 ? 1u : 0u;
    v.epoch = P.epoch;
    v.csrc = J.src_buf ? a.codes1 : a.codes0;
    v.cdst = J.src_buf ? a.codes0 : a.codes1;
    const uint32_t tid = threadIdx.x;
    if (tid < 8) sh.left_bins[tid] = J.left_bins[tid];  // visible after the first barrier below
    const uint32_t *bins32 = reinterpret_cast<const uint32_t *>(R.bins);
    if (v.hist)
        for (uint32_t k = tid; k < static_cast<uint32_t>(LDS_WORDS); k += 1024) lds[k] = 0;
    uint32_t dxs[4], dcols[DP ? DP : 1][4];
    if constexpr (DP > 0) dense_lanes<DP>(R.pos_word, tid & 63u, dxs, dcols);

    if (!v.partition) {
        // A later slab: the built child's rows as the partition launch (an earlier kernel) left them in dst, the left
        // child first-first from begin, the right one after the left rows (any order sums alike), a workgroup
        // taking an equal share; no tile is ranked again. Whenever flush_rows rows have gone into the packed words
        // they are added into the partial as {g, h} pairs; a workgroup that never flushes stores them packed.
        const uint32_t nb = v.built_left ? J.left : v.count - J.left;
        const uint32_t b0 = v.begin + (v.built_left ? 0u : J.left);
        const uint32_t per = (nb + v.groups - 1) / v.groups;
        const uint32_t c0 = min(nb, gi * per), c1 = min(nb, c0 + per);
        const uint32_t *list = v.dst + b0;
        const uint8_t *codes = CODES ? v.cdst + b0 : nullptr;
        int2 *pairs = reinterpret_cast<int2 *>(R.partial) + static_cast<size_t>(wg) * step_partial_stride(W);
        const uint32_t col_bins = (PACK > 1 || DP > 0) ? 256u : R.col_bins[tid % W];
        __syncthreads();  // the LDS histogram is zeroed
        bool flushed = false;
        for (uint32_t ca = c0; ca < c1;) {
            const uint32_t cb = c1 - ca < a.flush_rows ? c1 : ca + a.flush_rows;
            if (ca > c0) {
                flush_pairs<W, Q32>(lds, pairs, col_bins, flushed);
                flushed = true;
            }
            step_hist<W, WIDE, PACK, Q32, DP, UNROLL, 16, CODES>(lds, list, ca, cb, a.gh, bins32, a.dw_row, dxs, dcols,
                                                                threadIdx.x >> 6, codes);
            ca = cb;
        }
        if (!flushed && !Q32) {
            __syncthreads();
            store_packed_partial<W>(lds, R.partial + 2 * static_cast<size_t>(wg) * step_partial_stride(W));
            if (tid == 0) R.fmt[wg] = 1u;
            return;
        }
        flush_pairs<W, Q32>(lds, pairs, col_bins, flushed);
        if (tid == 0) R.fmt[wg] = 0u;
        return;
    }

    if (packed) {  // one tile; the partial is the LDS words themselves
        __syncthreads();
        if (tid == 0) sh.tile = v.partition ? atomicAdd(&J.ticket, 1u) : gi;
        __syncthreads();
        const uint32_t t = sh.tile;
        TileRows r;
        tile_rows<CODES>(v, t, r);
        tile_bins(v, r);
        TileState st;
        const uint32_t nb = tile_front<CODES>(v, t, r, st, sh);
        // wave 0 resolves the tile's offset while the other waves histogram it (wv: the wave, uniform)
        const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
        if (v.partition) {
            if (wv == 0) tile_lookback(v, a, t, st, sh);
            else if (v.hist) step_hist<W, WIDE, PACK, Q32, DP, 16, 15, CODES>(lds, sh.list, 0, nb, a.gh, bins32, a.dw_row, dxs, dcols, wv - 1, sh.codes);
        } else if (v.hist) {
            step_hist<W, WIDE, PACK, Q32, DP, 16, 16, CODES>(lds, sh.list, 0, nb, a.gh, bins32, a.dw_row, dxs, dcols, threadIdx.x >> 6, sh.codes);
        }
        __syncthreads();  // the offset and the histogram are complete
        if (v.partition) tile_scatter<CODES>(v, t, st, sh);
        if (!v.hist) return;
        if constexpr (Q32) {  // the counters as a {g, h} pair partial
            int2 *pairs = reinterpret_cast<int2 *>(R.partial) + static_cast<size_t>(wg) * step_partial_stride(W);
            flush_pairs<W, true>(lds, pairs, 256u, false);
            if (tid == 0) R.fmt[wg] = 0u;
            return;
        }
        store_packed_partial<W>(lds, R.partial + 2 * static_cast<size_t>(wg) * step_partial_stride(W));
        if (tid == 0) R.fmt[wg] = 1u;
        return;
    }

    // several tiles per workgroup: whenever flush_rows rows have gone into the packed words they are added into the
    // partial as {g, h} pairs; a workgroup that never flushes stores its partial packed instead
    int2 *pairs = reinterpret_cast<int2 *>(R.partial) + static_cast<size_t>(wg) * step_partial_stride(W);
    // slot tid + 1024 j is bin (tid + 1024 j) / W of column tid % W; a packed column's features are all stored
    const uint32_t col_bins = (PACK > 1 || DP > 0) ? 256u : R.col_bins[tid % W];
    uint32_t pending = 0;  // rows added to the packed LDS words since they were last flushed
    bool flushed = false;
    // partition launches take tiles in ticket order, the next ticket drawn while the current tile is worked on (a
    // look-back only ever waits on lower tiles, so holding a later one cannot block it); histogram-only launches
    // take tiles gi, gi + groups, ...
    // A workgroup holds the tickets of its current and next tiles, and loads the next tile's rows while it
    // histograms the current one (their split bins after it).
    // At most a.tile_cap tickets a workgroup, whatever the others' pace (its i32 sums; the planner gives every job
    // enough workgroups for its tiles at that many each).
    __syncthreads();  // the LDS histogram is zeroed
    uint32_t taken = 0;  // tickets this workgroup drew (thread 0's count)
    if (tid == 0) {
        sh.tile = v.partition ? atomicAdd(&J.ticket, 1u) : gi;
        sh.tile2 = v.partition ? (a.tile_cap > 1u ? atomicAdd(&J.ticket, 1u) : v.ntiles) : gi + v.groups;
        taken = a.tile_cap > 1u ? 2u : 1u;
    }
    __syncthreads();
    uint32_t t = sh.tile, tn = sh.tile2;
    uint32_t next = gi + 2 * v.groups;
    TileRows r;
    if (t < v.ntiles) {
        tile_rows<CODES>(v, t, r);
        tile_bins(v, r);
    }
    while (t < v.ntiles) {
        TileState st;
        const uint32_t nb = tile_front<CODES>(v, t, r, st, sh);
        uint32_t ticket = next;
        if (v.partition && tid == 0) {
            ticket = taken < a.tile_cap ? atomicAdd(&J.ticket, 1u) : v.ntiles;
            ++taken;
        }
        next += v.groups;
        if (tn < v.ntiles) tile_rows<CODES>(v, tn, r);
        // a tile that takes the packed words past flush_rows rows is histogrammed by all waves around the flushes
        // (block-wide); otherwise wave 0 resolves the tile's offset while the other waves histogram it
        const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
        bool hist_done = !v.hist;
        if (v.hist && pending + nb > a.flush_rows) {
            uint32_t c0 = 0;
            while (c0 < nb) {
                if (pending >= a.flush_rows) {
                    flush_pairs<W, Q32>(lds, pairs, col_bins, flushed);
                    pending = 0;
                    flushed = true;
                }
                uint32_t room = a.flush_rows - pending;
                uint32_t c1 = nb - c0 < room ? nb : c0 + room;
                step_hist<W, WIDE, PACK, Q32, DP, UNROLL, 16, CODES>(lds, sh.list, c0, c1, a.gh, bins32, a.dw_row, dxs, dcols, threadIdx.x >> 6, sh.codes);
                pending += c1 - c0;
                c0 = c1;
            }
            hist_done = true;
        }
        if (v.partition) {
            if (wv == 0) tile_lookback(v, a, t, st, sh);
            else if (!hist_done) step_hist<W, WIDE, PACK, Q32, DP, UNROLL, 15, CODES>(lds, sh.list, 0, nb, a.gh, bins32, a.dw_row, dxs, dcols, wv - 1, sh.codes);
            __syncthreads();  // the offset is in sh.prefix
            tile_scatter<CODES>(v, t, st, sh);
        } else if (!hist_done) {
            step_hist<W, WIDE, PACK, Q32, DP, UNROLL, 16, CODES>(lds, sh.list, 0, nb, a.gh, bins32, a.dw_row, dxs, dcols, threadIdx.x >> 6, sh.codes);
        }
        if (!hist_done) pending += nb;
        if (tn < v.ntiles) tile_bins(v, r);
        __syncthreads();  // the tile's list is consumed
        if (tid == 0) sh.tile = ticket;
        __syncthreads();
        t = tn;
        tn = sh.tile;
    }
    if (!v.hist) return;
    if (!flushed && !Q32) {  // every row still in the packed words: the partial is packed, as a one-tile workgroup's
        __syncthreads();
        store_packed_partial<W>(lds, R.partial + 2 * static_cast<size_t>(wg) * step_partial_stride(W));
        if (tid == 0) R.fmt[wg] = 1u;
        return;
    }
    flush_pairs<W, Q32>(lds, pairs, col_bins, flushed);
    if (tid == 0) R.fmt[wg] = 0u;
}

// CODES: the built rows' gradients come from the codes beside their ids (a.codes0 / a.codes1), else gathered. The
// two are separate instances: in one kernel behind a branch, the register allocator spilled both.
template <int W, bool WIDE = false, int PACK = 1, bool Q32 = false, int DP = 0, bool CODES = false>
__global__ __launch_bounds__(1024) void k_step_rows(StepArgs a) {
    __shared__ int32_t lds[step_lds_words<W, Q32, DP>()];
    __shared__ StepShared sh;
    step_rows_body<W, WIDE, PACK, Q32, DP, CODES>(a, lds, sh);
}

// Measurement only (profile mode): the distinct 128-byte lines (the size of every L2 miss's request to memory) a
// split step's gathers must touch, from the step's own plan and partition buffers, right after its k_step_rows
// launches. Per job, over the parent's rows (ascending in row id, whatever order they are stored in): the lines of
// the column-major split-feature array their bins lie in (128 rows a line, 64 for two-byte bins) and, over the built
// child's rows (sorted too), the lines of the packed gradient array (32 rows a line). A sorted run of rows touches as
// many lines as it has distinct row / rows-per-line values, so each is a count of the positions where that value
// changes. `shared`, when set, is one bit per (column-major feature, split-bin line), or-ed over every job of the
// step: the lines the step would touch if jobs that split on the same feature shared them. counters: [0] parent
// rows, [1] their split-bin lines, [2] built rows, [3] their gradient lines, [5] partials written (the first slab's
// workgroups of histogrammed jobs), [6] of those, packed (`fmt`: the first slab's partial formats), [7]-[9] parent
// rows, split-bin lines and built rows of the sparse jobs (fewer than two parent rows a split-bin line). grid: (x,
// JMAX); one block per job when `sparse_split` is needed (x = 1).
__global__ __launch_bounds__(256) void k_sector_model(const StepPlan *plan, const uint32_t *buf0, const uint32_t *buf1,
                                                      uint32_t col16, uint32_t *shared, uint64_t lines_per_col,
                                                      const uint32_t *fmt, unsigned long long *counters) {
    __shared__ unsigned long long part[4];
    const StepPlan &P = *plan;
    const uint32_t j = blockIdx.y;
    if (threadIdx.x < 4) part[threadIdx.x] = 0;
    if (j < P.njobs && blockIdx.x == 0 && threadIdx.x == 0 && P.jobs[j].hist) {
        const JobPlan &J = P.jobs[j];
        unsigned long long packed = 0;
        for (uint32_t k = 0; k < J.groups; ++k) packed += fmt[J.group_base + k] ? 1ull : 0ull;
        atomicAdd(counters + 5, static_cast<unsigned long long>(J.groups));
        atomicAdd(counters + 6, packed);
    }
    __syncthreads();
    if (j < P.njobs) {
        const JobPlan &J = P.jobs[j];
        const uint32_t *src = J.src_buf ? buf1 : buf0, *dst = J.src_buf ? buf0 : buf1;
        const uint32_t sshift = col16 ? 6u : 7u;
        unsigned long long prow = 0, psec = 0, brow = 0, bsec = 0;
        for (uint32_t i = threadIdx.x; i < J.count; i += blockDim.x) {
            const uint32_t at = J.src_rev ? J.begin + J.count - 1 - i : J.begin + i;
            const uint32_t r = src[at];
            ++prow;
            if (i == 0 || (src[J.src_rev ? at + 1 : at - 1] >> sshift) != (r >> sshift)) ++psec;
            if (shared) {
                const uint64_t bit = static_cast<uint64_t>(J.col) * lines_per_col + (r >> sshift);
                atomicOr(shared + (bit >> 5), 1u << (bit & 31u));
            }
        }
        if (J.hist) {
            // the built child: the left one first-first at begin, the right one last-first after the left rows
            const uint32_t b = J.built_side == 0 ? J.begin : J.begin + J.left;
            const uint32_t n = J.built_side == 0 ? J.left : J.count - J.left;
            for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
                const uint32_t r = dst[b + i];
                ++brow;
                if (i == 0 || (dst[b + i - 1] >> 5) != (r >> 5)) ++bsec;
            }
        }
        atomicAdd(&part[0], prow);
        atomicAdd(&part[1], psec);
        atomicAdd(&part[2], brow);
        atomicAdd(&part[3], bsec);
    }
    __syncthreads();
    if (threadIdx.x < 4 && part[threadIdx.x]) atomicAdd(counters + threadIdx.x, part[threadIdx.x]);
    if (threadIdx.x == 0 && part[1] * 2 > part[0]) {  // a sparse job (one block a job)
        atomicAdd(counters + 7, part[0]);
        atomicAdd(counters + 8, part[1]);
        atomicAdd(counters + 9, part[2]);
    }
}

// Measurement only: the set bits of k_sector_model's shared-line bitmap into counters[4], the bitmap cleared.
__global__ __launch_bounds__(256) void k_sector_bits(uint32_t *bits, uint64_t words, unsigned long long *counters) {
    unsigned long long c = 0;
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < words;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint32_t w = bits[i];
        if (w) {
            c += static_cast<unsigned long long>(__popc(w));
            bits[i] = 0;
        }
    }
    for (int o = 32; o > 0; o >>= 1) c += static_cast<unsigned long long>(__shfl_xor(static_cast<long long>(c), o));
    if ((threadIdx.x & 63u) == 0 && c) atomicAdd(counters + 4, c);
}

// Four columns of one slab: a work unit of k_step_reduce and k_step_scan.
struct ColGroup {
    uint64_t partial;  // the slab's partials, in {g, h} pairs from the start of the step partial buffer
    uint32_t width;    // the slab's W
    uint32_t c0;       // first column of the group in the slab
    uint32_t fmt;      // the slab's first k_step_rows workgroup in the partial-format flags
    uint32_t offset[4][4];  // per segment and column: its feature's first bin in the flat histogram
    uint32_t bins[4][4];    // per segment and column: the feature's bins (0 for padding)
    uint32_t stride[4];     // per column: flat-histogram bins between its consecutive bins (4 in a wide slab)
    uint32_t seg_shift;     // a column holds a feature each 2^seg_shift bins (8: one; 7 or 6 in a packed slab)
    uint32_t dense;         // a dense slab: the slots' flat bins come from the slot table at slot_base
    uint32_t slot_base;
};

// Block-wide hand-off through `counter`: true in every thread of the block that arrives last of `target` blocks,
// which then sees the global stores every arriving block made before arriving; that block returns the counter
// to 0. Each thread first waits for its own stores to reach L2, so thread 0's release fence (an L2 write-back,
// waited for before the increment) covers the whole block, and its acquire fence covers the last block's reads.
__device__ __forceinline__ bool arrive_last(uint32_t *counter, uint32_t target) {
    __shared__ uint32_t s_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __builtin_amdgcn_s_waitcnt(0);
        bool last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == target - 1u;
        if (last) {
            __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        s_last = last ? 1u : 0u;
    }
    __syncthreads();
    return s_last != 0;
}

// A scan unit is one wave's scan of a child: one feature (SEGL 64), or 4 features of at most 64 bins (SEGL 16) or
// 16 of at most 16 bins (SEGL 4), a segment of lanes each (UNIT_FEATS entries a unit).
struct ScanStepArgs {
    const int32_t *unit_feat;   // per scan unit, UNIT_FEATS numerical features (segment order), -1 for padding
    const uint32_t *unit_segl;  // per scan unit, its lanes a feature: 64, 16 or 4
    uint32_t nseg;              // the units of several features come first
    const uint32_t *cat_feats;  // the categorical features (k_step_cat)
    uint32_t ncat;
    StepPlan *plan;
};

struct SelectArgs {
    uint32_t *all_count;        // jobs selected; returned to 0 by the last one
    StepPlan *plan;             // this step's plan
    StepPlan *next;             // the next step's
};

struct ReduceStepArgs {
    const int32_t *partial;     // the step partial buffer
    const uint32_t *fmt;        // the partials' formats (per slab, per k_step_rows workgroup: 1 packed, 0 pairs)
    const ColGroup *cgs;        // [ncg]
    StepPlan *plan;
    const uint32_t *slot_flat;  // dense slabs: per slot, its flat-histogram bin + 1 (0: none)
};

// The end of job j, by one block (learner.rs:294-352): both children's best splits from their per-feature
// candidates (split.rs:866-880), then their leaves in the speculative tree and the job's leaf marked expanded (thread
// 0). Up to 256 features, waves 0 and 1 take a child each while wave 2 counts the job's evaluated features; beyond,
// half the block's waves take a child, each over a share of the features, and their bests are merged (the (gain,
// feature) order is total, so any split of the features gives the same winner), every wave counting a share of the
// evaluated features: one wave a child took 2000 features in 32 rounds of dependent loads, and the merge's extra
// barrier costs small feature counts 1 us a step.
__device__ void job_select(const GrowState &g, const JobPlan &J, uint32_t j) {
    __shared__ SplitOut s_out[2];
    __shared__ uint32_t s_used;
    __shared__ double s_wb[2][8];
    __shared__ int s_wf[2][8];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    GrowCtl *ctl = g.ctl;
    const int64_t left = static_cast<int64_t>(J.left);
    const int64_t right = J.parent_count - left;
    if (!(left > 0 && right > 0)) {  // uniform over the block
        if (threadIdx.x == 0) {
            ctl->error = 1;
            ctl->done = 1;
            const uint32_t info[8] = {j, J.t, J.count, J.left, J.ntiles, J.groups, J.packed, 0u};
            for (int k = 0; k < 8; ++k) ctl->err_info[k] = info[k];
        }
        return;
    }
    const int32_t kid = J.kid;
    const int32_t depth = g.tl[J.t].depth + 1;
    const int64_t min_pair = 2 * g.cfg.min_data_in_leaf;
    const bool searched = J.hist && depth_allows(g, depth) && (left >= min_pair || right >= min_pair);
    const uint32_t nw = blockDim.x >> 6;
    if (g.nf <= 256u || nw < 4u) {  // uniform
        // waves 0 and 1: the best split of the left and the right child; wave 2: the job's evaluated features
        // (learner.rs:262-265), for the byte count
        if (wave == 2) {
            const uint8_t *prow = g.splittable + static_cast<size_t>(J.t) * g.nf;
            uint32_t used = 0;
            for (uint32_t f = lane; f < g.nf; f += 64u)
                used += static_cast<uint32_t>(__popcll(__ballot(g.mask[f] != 0 && prow[f] != 0)));
            if (lane == 0) s_used = used;
        } else if (wave < 2) {
            const uint32_t ch = wave;
            SplitOut out = {};
            if (searched) {
                const FeatCand *cands = g.cands + (static_cast<size_t>(j) * 2 + ch) * g.nf;
                uint8_t *row = g.splittable + static_cast<size_t>(kid + static_cast<int32_t>(ch)) * g.nf;
                double best = 0.0;
                int bf = -1;
                for (uint32_t f = lane; f < g.nf; f += 64u) {
                    const FeatCand &c = cands[f];
                    row[f] = static_cast<uint8_t>(c.splittable);
                    if (!c.found) continue;
                    const double gv = (c.gain != c.gain) ? -__builtin_inf() : c.gain;
                    if (cand_better(gv, static_cast<int>(f), best, bf)) {
                        best = gv;
                        bf = static_cast<int>(f);
                    }
                }
                wave_best(best, bf);
                if (bf >= 0) {  // the winner, read once more where the scans left it
                    const int64_t cnt = ch == 0 ? left : right;
                    out = split_out(cands[bf], bf, make_ctx(g.cfg, grow_sg(g), grow_sh(g), J.child_ug[ch], J.child_uh[ch], cnt), g.cfg);
                }
            }
            if (lane == 0) s_out[ch] = out;
        }
        __syncthreads();
    } else {
        // the job's evaluated features (learner.rs:262-265), for the byte count, a share a wave
        const uint32_t wpc = nw >> 1 < 8u ? nw >> 1 : 8u;  // waves a child
        if (threadIdx.x == 0) s_used = 0;
        __syncthreads();
        {
            const uint8_t *prow = g.splittable + static_cast<size_t>(J.t) * g.nf;
            uint32_t used = 0;
            for (uint32_t f = threadIdx.x; f < g.nf; f += blockDim.x) used += g.mask[f] != 0 && prow[f] != 0 ? 1u : 0u;
            used = wave_total(used);
            if (lane == 0 && used) atomicAdd(&s_used, used);
        }
        // waves c wpc .. c wpc + wpc - 1: child c's best over features sub 64 + lane, + 64 wpc, ...
        if (wave < 2u * wpc && searched) {
            const uint32_t ch = wave / wpc, sub = wave - ch * wpc;
            const FeatCand *cands = g.cands + (static_cast<size_t>(j) * 2 + ch) * g.nf;
            uint8_t *row = g.splittable + static_cast<size_t>(kid + static_cast<int32_t>(ch)) * g.nf;
            double best = 0.0;
            int bf = -1;
            for (uint32_t f = sub * 64u + lane; f < g.nf; f += 64u * wpc) {
                const FeatCand &c = cands[f];
                row[f] = static_cast<uint8_t>(c.splittable);
                if (!c.found) continue;
                const double gv = (c.gain != c.gain) ? -__builtin_inf() : c.gain;
                if (cand_better(gv, static_cast<int>(f), best, bf)) {
                    best = gv;
                    bf = static_cast<int>(f);
                }
            }
            wave_best(best, bf);
            if (lane == 0) {
                s_wb[ch][sub] = best;
                s_wf[ch][sub] = bf;
            }
        }
        __syncthreads();
        // waves 0 and 1: the left and the right child's winner over its waves' bests
        if (wave < 2) {
            const uint32_t ch = wave;
            SplitOut out = {};
            if (searched) {
                double wb = lane < wpc ? s_wb[ch][lane] : 0.0;
                int wf = lane < wpc ? s_wf[ch][lane] : -1;
                wave_best(wb, wf);
                if (wf >= 0) {  // the winner, read once more where the scans left it
                    const FeatCand *cands = g.cands + (static_cast<size_t>(j) * 2 + ch) * g.nf;
                    const int64_t cnt = ch == 0 ? left : right;
                    out = split_out(cands[wf], wf, make_ctx(g.cfg, grow_sg(g), grow_sh(g), J.child_ug[ch], J.child_uh[ch], cnt), g.cfg);
                }
            }
            if (lane == 0) s_out[ch] = out;
        }
        __syncthreads();
    }
    // the children's best splits, copied a dword a thread (no child-sized copy through one thread's stack)
    static_assert(sizeof(SplitOut) % 4 == 0 && sizeof(SplitOut) / 4 <= 64, "a split copies in one wave");
    if (threadIdx.x < 128) {
        const uint32_t ch = threadIdx.x >> 6, d = threadIdx.x & 63u;
        if (d < sizeof(SplitOut) / 4)
            reinterpret_cast<uint32_t *>(&g.tl[kid + static_cast<int32_t>(ch)].best)[d] =
                reinterpret_cast<const uint32_t *>(&s_out[ch])[d];
    }
    if (threadIdx.x == 0) {
        const SplitOut &info = g.tl[J.t].best;
        const uint32_t has[2] = {s_out[0].found ? 1u : 0u, s_out[1].found ? 1u : 0u};
        const double gain[2] = {s_out[0].gain, s_out[1].gain};
        const double lv = info.left_output, rv = info.right_output;
        const double lh = info.left_hess, rh = info.right_hess;
#pragma unroll
        for (uint32_t ch = 0; ch < 2; ++ch) {
            TLeaf &c = g.tl[kid + static_cast<int32_t>(ch)];
            c.begin = ch == 0 ? J.begin : J.begin + J.left;
            c.count = ch == 0 ? J.left : J.count - J.left;
            c.ug = ch == 0 ? info.left_grad : info.right_grad;
            c.uh = ch == 0 ? lh : rh;
            c.cnt = ch == 0 ? left : right;
            // the built child's histogram goes to the job's new slot, the other child keeps its parent's
            c.slot = searched ? ((J.built_side == ch) ? J.built_slot : J.parent_slot) : -1;
            c.has_best = searched ? has[ch] : 0u;
            c.buf = 1u - J.src_buf;
            c.rev = ch;  // the split step writes the left child first-first and the right child last-first
            c.depth = depth;
            c.state = T_LEAF;
            c.kid = -1;
            c.pad_ = 0;
            const double v = ch == 0 ? lv : rv;
            c.value = v != v ? 0.0 : v;
            c.weight = (ch == 0 ? lh : rh) * grow_sh(g);
            g.tk[kid + static_cast<int32_t>(ch)] = TKey{gain[ch], searched ? has[ch] : 0u, T_LEAF, -1, 0u};
        }
        g.tl[J.t].state = T_EXPANDED;
        g.tk[J.t].state = T_EXPANDED;
        if (J.hist) {  // the built child's histogram was made, searched or not
            const double built_rows = J.built_side == 0 ? static_cast<double>(left) : static_cast<double>(right);
            atomicAdd(&ctl->hist_rows, built_rows);
            atomicAdd(&ctl->hist_bins, built_rows * static_cast<double>(s_used));
            atomicAdd(&ctl->hist_builds, 1.0);
        }
        atomicAdd(&ctl->part_rows, static_cast<double>(J.count));
    }
}

// The built child's histogram of each job from its workgroups' partials, and its sibling's by subtraction in place
// of the parent's (learner.rs:356-371). Work items (job, column group, bin range) in a grid-stride loop: a thread
// adds one stripe of the workgroups' partials of one bin of the group's four columns, reading each partial in its
// own format (packed: one 16-byte load; {g, h} pairs: two), and the stripes meet in LDS. grid: any, 256 threads.
// One child's candidate of numerical feature sf in job j (split.rs:584-620), on one wave: the feature scanned in both
// directions over the child's histogram (the built one, or the sibling the reduce formed in the parent's slot).
template <bool WIDE>
__device__ __forceinline__ void scan_child(const GrowState &g, const JobPlan &J, uint32_t j, int32_t sf, const FeatDev &sm,
                                           uint32_t child) {
    const uint32_t lane = threadIdx.x & 63u;
    const bool sev = g.mask[sf] != 0 && g.splittable[static_cast<size_t>(J.t) * g.nf + sf] != 0;
    const int64_t *hist = g.pool + static_cast<size_t>(child == J.built_side ? J.built_slot : J.parent_slot) * g.slot_stride;
    const int64_t cnt = child == 0 ? static_cast<int64_t>(J.left) : J.parent_count - static_cast<int64_t>(J.left);
    const Ctx c = make_ctx(g.cfg, grow_sg(g), grow_sh(g), J.child_ug[child], J.child_uh[child], cnt);
    FeatCand r = {};
    if (scan_searched(c, sm, sev)) {
        Grown rg = {}, fg = {};
        bool rf, ff;
        if constexpr (WIDE) scan_numerical_wide(c, g.cfg, sm, hist, rf, rg, ff, fg);
        else scan_numerical(c, g.cfg, sm, hist, rf, rg, ff, fg);
        r = feature_candidate(c, sm, rf, rg, ff, fg);
    }
    if (lane == 0) g.cands[(static_cast<size_t>(j) * 2 + child) * g.nf + sf] = r;
}

__global__ __launch_bounds__(256) void k_step_reduce(GrowState g, ReduceStepArgs a) {
    __shared__ int64_t red[8][256];  // the stripes' sums, [value][thread]: conflict-free
    const StepPlan &P = *a.plan;  // empty once the tree is done (k_step_select)
    const uint32_t tid = threadIdx.x;
    for (uint32_t item = blockIdx.x; item < P.total_red; item += gridDim.x) {
        const uint32_t j = job_of(P.red_base, P.njobs, item);
        const JobPlan &J = P.jobs[j];
        const uint32_t ways = J.ways, groups = J.groups;
        const uint32_t r = item - J.red_base;
        uint32_t cgi, sub;
        if ((g.ncg & 15u) == 0u) {
            // column groups 2p and 2p + 1 (one 128-byte line of a packed partial) 8 items apart, so on one XCD (blocks
            // go to the 8 XCDs in turn): the second reads the line from that XCD's L2
            const uint32_t w = r & 15u, pi = (r >> 4) * 8u + (w & 7u), pair = pi / ways;
            sub = pi - pair * ways;
            cgi = 2u * pair + (w >> 3);
        } else {
            cgi = r / ways;
            sub = r - cgi * ways;
        }
        const ColGroup &cg = a.cgs[cgi];  // read in place: a column is picked per thread
        int64_t *built = g.pool + static_cast<size_t>(J.built_slot) * g.slot_stride;
        int64_t *parent = g.pool + static_cast<size_t>(J.parent_slot) * g.slot_stride;
        const size_t stride4 = step_partial_stride(cg.width) / 2;  // int4s from one partial to the next
        const uint32_t ns = 256u / ways;                           // the item's bins
        const uint32_t q = tid / ns;                               // this thread's stripe
        const uint32_t bin = sub * ns + tid % ns;
        // bin `bin` of the group's columns in a partial: packed, int4 (bin / 4) * W + c0 + bin % 4; pairs, the int4s
        // at (bin * W + c0) / 2 and the next
        const int4 *src = reinterpret_cast<const int4 *>(a.partial + 2 * cg.partial) + static_cast<size_t>(J.group_base) * stride4;
        const size_t po = static_cast<size_t>(bin / 4u) * cg.width + cg.c0 + bin % 4u;
        const size_t qo = (static_cast<size_t>(bin) * cg.width + cg.c0) / 2;
        const uint32_t *fmt = a.fmt + cg.fmt + J.group_base;
        // the parent's bins are loaded with the partials (the writes below need them); every partial is first read
        // as packed, and a {g, h} pair partial (a workgroup that flushed) is read again in its own layout
        const uint32_t seg = bin >> cg.seg_shift, vb = bin & ((1u << cg.seg_shift) - 1u);
        // the flat bin + 1 of each of the four columns' slot (0: none)
        uint32_t fl[4];
        if (cg.dense) {
            const uint4 t = *reinterpret_cast<const uint4 *>(a.slot_flat + cg.slot_base + static_cast<size_t>(bin) * cg.width + cg.c0);
            fl[0] = t.x;
            fl[1] = t.y;
            fl[2] = t.z;
            fl[3] = t.w;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) fl[c] = vb < cg.bins[seg][c] ? cg.offset[seg][c] + vb * cg.stride[c] + 1u : 0u;
        }
        int64_t pg[4] = {0, 0, 0, 0}, ph[4] = {0, 0, 0, 0};
        if (q == 0) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if (fl[c]) {
                    const size_t o = 2 * static_cast<size_t>(fl[c] - 1u);
                    pg[c] = parent[o];
                    ph[c] = parent[o + 1];
                }
            }
        }
        int64_t sg[4] = {0, 0, 0, 0}, sh[4] = {0, 0, 0, 0};
        for (uint32_t w = q; w < groups; w += 8u * ways) {
            bool pk[8];
            int4 x[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t wk = w + k * ways;
                const uint32_t wc = wk < groups ? wk : q;
                pk[k] = fmt[wc] != 0u;
                x[k] = src[static_cast<size_t>(wc) * stride4 + po];
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t wk = w + k * ways;
                if (wk >= groups) continue;
                if (pk[k]) {
                    const int32_t v4[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int32_t gq = packed_g(v4[c]);
                        sg[c] += gq;
                        sh[c] += packed_h(v4[c], gq);
                    }
                } else {
                    const int4 *p = src + static_cast<size_t>(wk) * stride4;
                    const int4 a0 = p[qo], a1 = p[qo + 1];
                    sg[0] += a0.x;
                    sh[0] += a0.y;
                    sg[1] += a0.z;
                    sh[1] += a0.w;
                    sg[2] += a1.x;
                    sh[2] += a1.y;
                    sg[3] += a1.z;
                    sh[3] += a1.w;
                }
            }
        }
        if (ways > 1u) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                red[2 * c][tid] = sg[c];
                red[2 * c + 1][tid] = sh[c];
            }
            __syncthreads();
            if (q == 0)
                for (uint32_t k = 1; k < ways; ++k) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        sg[c] += red[2 * c][tid + k * ns];
                        sh[c] += red[2 * c + 1][tid + k * ns];
                    }
                }
        }
        if (q == 0) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if (fl[c]) {
                    const size_t o = 2 * static_cast<size_t>(fl[c] - 1u);
                    built[o] = sg[c];
                    built[o + 1] = sh[c];
                    parent[o] = pg[c] - sg[c];
                    parent[o + 1] = ph[c] - sh[c];
                }
            }
        }
        __syncthreads();  // the LDS is free for the next item
    }
}

// Scan items (job, unit, child), a wave each in a grid-stride loop: the unit's numerical feature scanned in both
// directions (split.rs:584-620) and its candidate written. Categorical features are k_step_cat's; features of
// two-byte bins are k_step_scan<true>'s, the others k_step_scan<false>'s. grid: any, 256 threads.
template <bool WIDE>
__global__ __launch_bounds__(256, WIDE ? 1 : 4) void k_step_scan(GrowState g, ScanStepArgs a) {
    const StepPlan &P = *a.plan;  // empty once the tree is done (k_step_select)
    const uint32_t total = P.total_scan * 2u;  // scan items count units: a wave per unit and child
    for (uint32_t item = blockIdx.x * 4u + (threadIdx.x >> 6); item < total; item += gridDim.x * 4u) {
        const uint32_t gi = item >> 1, child = item & 1u;
        const uint32_t j = job_of(P.scan_base, P.njobs, gi);
        const JobPlan &J = P.jobs[j];
        const uint32_t u = gi - J.scan_base;
        if (u < a.nseg) continue;  // k_step_scan_seg's
        const int32_t sf = a.unit_feat[u * UNIT_FEATS];
        if (sf < 0) continue;
        const FeatDev sm = g.feats[sf];
        if (sm.kind == 2 || (sm.wide != 0) != WIDE) continue;  // the other instantiation's, or k_step_cat's
        scan_child<WIDE>(g, J, j, sf, sm, child);
    }
}

// The scan units of several byte features a wave (k_step_scan's items of 16 or 4 lanes a feature): every segment
// scans (its shuffles take the whole wave), a padding or unsearched one keeping nothing. Its own kernel, so that the
// wave-wide scan keeps its registers (and occupancy). grid: any, 256 threads.
__global__ __launch_bounds__(256) void k_step_scan_seg(GrowState g, ScanStepArgs a) {
    const StepPlan &P = *a.plan;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t total = P.total_scan * 2u;
    for (uint32_t item = blockIdx.x * 4u + (threadIdx.x >> 6); item < total; item += gridDim.x * 4u) {
        const uint32_t gi = item >> 1, child = item & 1u;
        const uint32_t j = job_of(P.scan_base, P.njobs, gi);
        const JobPlan &J = P.jobs[j];
        const uint32_t u = gi - J.scan_base;
        if (u >= a.nseg) continue;  // k_step_scan's
        const uint32_t segl = a.unit_segl[u];  // 16 or 4, wave-uniform
        const uint32_t t = lane & (segl - 1u);
        const int32_t sf = a.unit_feat[u * UNIT_FEATS + lane / segl];
        const FeatDev sm = sf >= 0 ? g.feats[sf] : FeatDev{};
        const bool sev = sf >= 0 && g.mask[sf] != 0 && g.splittable[static_cast<size_t>(J.t) * g.nf + sf] != 0;
        const int64_t *hist = g.pool + static_cast<size_t>(child == J.built_side ? J.built_slot : J.parent_slot) * g.slot_stride;
        const int64_t cnt = child == 0 ? static_cast<int64_t>(J.left) : J.parent_count - static_cast<int64_t>(J.left);
        const Ctx c = make_ctx(g.cfg, grow_sg(g), grow_sh(g), J.child_ug[child], J.child_uh[child], cnt);
        Grown rg = {}, fg = {};
        bool rf = false, ff = false;
        if (segl == 16u) scan_numerical<16>(c, g.cfg, sm, hist, rf, rg, ff, fg);
        else scan_numerical<4>(c, g.cfg, sm, hist, rf, rg, ff, fg);
        FeatCand r = {};
        if (sf >= 0 && scan_searched(c, sm, sev)) r = feature_candidate(c, sm, rf, rg, ff, fg);
        if (t == 0 && sf >= 0) g.cands[(static_cast<size_t>(j) * 2 + child) * g.nf + sf] = r;
    }
}

// The categorical features' candidates of every job (split.rs:694-844): a wave per (job, feature, child) in a
// grid-stride loop. grid: any, 256 threads.
__global__ __launch_bounds__(256) void k_step_cat(GrowState g, ScanStepArgs a) {
    __shared__ CatScratch cats[4];
    const StepPlan &P = *a.plan;  // empty once the tree is done (k_step_select)
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t per_job = 2 * a.ncat, total = P.njobs * per_job;
    for (uint32_t item = blockIdx.x * 4 + wave; item < total; item += gridDim.x * 4) {
        const uint32_t j = item / per_job, r = item - j * per_job, child = r & 1u;
        const JobPlan &J = P.jobs[j];
        if (!J.hist) continue;
        const uint32_t f = a.cat_feats[r >> 1];
        const FeatDev sm = g.feats[f];
        const bool sev = g.mask[f] != 0 && g.splittable[static_cast<size_t>(J.t) * g.nf + f] != 0;
        const int64_t *hist = g.pool + static_cast<size_t>(child == J.built_side ? J.built_slot : J.parent_slot) * g.slot_stride;
        const int64_t cnt = child == 0 ? static_cast<int64_t>(J.left) : J.parent_count - static_cast<int64_t>(J.left);
        const Ctx c = make_ctx(g.cfg, grow_sg(g), grow_sh(g), J.child_ug[child], J.child_uh[child], cnt);
        FeatCand out = {};
        if (scan_searched(c, sm, sev)) out = categorical_candidate(c, g.cfg, sm, hist, cats[wave], nullptr);
        if (lane == 0) g.cands[(static_cast<size_t>(j) * 2 + child) * g.nf + f] = out;
    }
}

// Block j selects both children of job j (job_select); the last block to finish runs advance. grid: jcap blocks.
template <uint32_t MAXL>
__global__ __launch_bounds__(512) void k_step_select(GrowState g, SelectArgs a) {
    __shared__ __align__(16) uint8_t scratch[sizeof(AdvShared<MAXL>)];
    // the next plan stays empty unless advance writes it (it runs after every block has arrived, so after this):
    // the steps after a finished tree do nothing without reading the control block
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.next->njobs = 0;
        a.next->total_groups = 0;
        a.next->total_red = 0;
        a.next->total_scan = 0;
    }
    if (g.ctl->done) return;
    StepPlan &P = *a.plan;
    const uint32_t j = blockIdx.x;
    if (j >= P.njobs) return;
    job_select(g, P.jobs[j], j);
    if (!arrive_last(a.all_count, P.njobs)) return;
    advance<MAXL>(g, *a.next, scratch);
}

}  // namespace srocm
