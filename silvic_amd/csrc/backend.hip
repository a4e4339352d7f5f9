// backend.hip - the C ABI of include/silvic_rocm.h on one MI355X (gfx950).
//
// One context owns one device, one stream (default priority) and the training data in its own layout:
//   - slabs: runs of up to 128 non-trivial features stored as W-byte rows (W = 32, 64 or 128), the layout the
//     histogram kernel reads (a scattered row of a 128-feature slab is one 128-byte line);
//   - column-major bins (one byte per row per feature), which partition and add_tree read;
//   - gradients, packed quantized gradients, two partition buffers and the per-leaf histogram pool.
// Host code mirrors silvic-core's Backend, Learner and Trainer (file:line beside each function); every
// histogram, subtraction, split scan, partition, quantization and score update runs on the device.

#include "../../include/silvic_rocm.h"
#include "kernels.hpp"
#include "lambdarank.hpp"
#include "rank_kernels.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>
#include <thread>
#include <functional>
#include <vector>

// The scratch of srocm_histogram_noalloc, the entry point that allocates nothing: the per-workgroup partial
// histograms its k_hist launches write in full and its k_hist_reduce reads. Every GPU the library runs on holds its
// own copy until the process ends. Host code never passes this name to a kernel or a copy: it uses the address
// hipGetSymbolAddress returned for the device (scratch_address), resolved once per device at srocm_create.
constexpr size_t NOALLOC_SCRATCH_PAIRS = size_t(2) << 20;  // {g, h} i32 pairs: 16 MiB
static __device__ __align__(256) int2 scratch[NOALLOC_SCRATCH_PAIRS];

namespace {

using namespace srocm;

struct Failure : std::runtime_error {
    int kind;
    Failure(int k, const std::string &m) : std::runtime_error(m), kind(k) {}
};

[[noreturn]] void fail(int kind, const std::string &m) { throw Failure(kind, m); }

void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) fail(SROCM_ERR_DEVICE, std::string("hip ") + what + ": " + hipGetErrorString(e));
}

void launch_check(const char *what) { hip_check(hipGetLastError(), what); }

// scratch's address on each device, resolved with that device current (each GPU holds its own copy of the array)
std::mutex g_scratch_mu;
std::vector<int2 *> g_scratch_at;

int2 *scratch_address(int dev) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_at.size() <= static_cast<size_t>(dev)) g_scratch_at.resize(static_cast<size_t>(dev) + 1, nullptr);
    if (!g_scratch_at[dev]) {
        void *p = nullptr;
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "scratch address");
        if (!p) fail(SROCM_ERR_DEVICE, "hip scratch address: null");
        g_scratch_at[dev] = static_cast<int2 *>(p);
    }
    return g_scratch_at[dev];
}

template <typename T>
struct DevBuf {
    T *p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    DevBuf(DevBuf &&o) noexcept : p(o.p), n(o.n) {
        o.p = nullptr;
        o.n = 0;
    }
    DevBuf &operator=(DevBuf &&o) noexcept {
        release();
        p = o.p;
        n = o.n;
        o.p = nullptr;
        o.n = 0;
        return *this;
    }
    ~DevBuf() { release(); }
    void alloc(size_t count) {
        if (p && count <= n) return;
        release();
        hip_check(hipMalloc(reinterpret_cast<void **>(&p), std::max<size_t>(count, 1) * sizeof(T)), "hipMalloc");
        n = count;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
};

template <typename T>
struct Pinned {
    T *p = nullptr;
    size_t n = 0;
    Pinned() = default;
    Pinned(const Pinned &) = delete;
    Pinned &operator=(const Pinned &) = delete;
    ~Pinned() { release(); }
    void alloc(size_t count) {
        if (p && count <= n) return;
        release();
        hip_check(hipHostMalloc(reinterpret_cast<void **>(&p), std::max<size_t>(count, 1) * sizeof(T), hipHostMallocDefault),
                  "hipHostMalloc");
        n = count;
    }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        n = 0;
    }
};

uint32_t div_up(uint64_t a, uint64_t b) { return static_cast<uint32_t>((a + b - 1) / b); }

// The split steps' planner gives a job k_step_rows workgroups in proportion to its tiles, each costing 1 in a dense
// leaf and up to 1 + STEP_SPARSE_WEIGHT in one sparser than a row a 128-byte line of split bins, plus
// STEP_HIST_WEIGHT a tile's worth of built-child rows (a fit of measured workgroup times on the 10M x 128 binary
// workload: 9.1 us a partitioned tile, 5.4 us more at the sparsest, 24.0 us a tile of built rows, R^2 0.97).
constexpr float STEP_HIST_WEIGHT = 2.63f, STEP_SPARSE_WEIGHT = 0.59f;

// ---------------------------------------------------------------------------------------------------------
// Host restatements the driver needs (quantize.rs, split.rs, tree.rs)
// ---------------------------------------------------------------------------------------------------------

inline uint32_t mix32_h(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

inline float uniform_h(uint32_t seed, uint32_t stream, uint32_t iteration, uint64_t row) {
    uint32_t row_hash = mix32_h(static_cast<uint32_t>(row) ^ mix32_h(static_cast<uint32_t>(row >> 32)));
    uint32_t h = mix32_h(seed ^ mix32_h(stream ^ mix32_h(iteration ^ row_hash)));
    return static_cast<float>(h >> 8) * (1.0f / 16777216.0f);
}

inline int64_t sat_i64_h(double x) {
    if (std::isnan(x)) return 0;
    if (x >= 9223372036854775807.0) return std::numeric_limits<int64_t>::max();
    if (x <= -9223372036854775808.0) return std::numeric_limits<int64_t>::min();
    return static_cast<int64_t>(x);
}

inline double positive_or_one(double v) { return (v > 0.0 && std::isfinite(v)) ? v : 1.0; }

// quantize.rs:56-84
srocm_quant_spec make_quant_spec(double max_abs_grad, double max_hess, bool constant_hessian, double constant,
                                 uint32_t num_bins, bool stochastic, uint32_t seed, uint32_t iteration) {
    srocm_quant_spec s{};
    s.grad_max_q = static_cast<int32_t>(num_bins / 2);
    s.hess_max_q = static_cast<int32_t>(num_bins);
    s.grad_scale = positive_or_one(max_abs_grad / static_cast<double>(s.grad_max_q));
    s.hess_scale = constant_hessian ? positive_or_one(constant) : positive_or_one(max_hess / static_cast<double>(s.hess_max_q));
    s.inv_grad_scale = static_cast<float>(1.0 / s.grad_scale);
    s.inv_hess_scale = static_cast<float>(1.0 / s.hess_scale);
    s.constant_hessian = constant_hessian;
    s.stochastic = stochastic;
    s.seed = seed;
    s.iteration = iteration;
    return s;
}

// quantize.rs:153-159
float fixed_point_scale(double max_abs) {
    if (!std::isfinite(max_abs) || max_abs <= 0.0) return 1.0f;
    int32_t e = 30 - static_cast<int32_t>(sat_i64_h(std::ceil(std::log2(max_abs))));
    e = std::clamp(e, -126, 127);
    return std::ldexp(1.0f, e);
}

// split.rs:145-154, 190-192
inline double leaf_output_h(double g, double h, double l1, double l2) {
    double reg = std::fmax(std::fabs(g) - l1, 0.0);
    double sign = static_cast<double>(static_cast<int>(g > 0.0) - static_cast<int>(g < 0.0));
    return -(sign * reg) / (h + l2);
}

inline int total_cmp_f(float a, float b) {
    int32_t x, y;
    std::memcpy(&x, &a, 4);
    std::memcpy(&y, &b, 4);
    x ^= static_cast<int32_t>(static_cast<uint32_t>(x >> 31) >> 1);
    y ^= static_cast<int32_t>(static_cast<uint32_t>(y >> 31) >> 1);
    return (x > y) - (x < y);
}

constexpr double K_EPS_H = static_cast<double>(1e-15f);
constexpr double ZERO_THRESHOLD = static_cast<double>(1e-35f);  // tree.rs:13
inline double nan_to_zero(double v) { return std::isnan(v) ? 0.0 : v; }
inline double round_to_zero(double v) { return std::fabs(v) > ZERO_THRESHOLD ? v : 0.0; }

// tree.rs:46-203, thresholds as bins
struct HostTree {
    uint32_t num_leaves = 1;
    std::vector<int32_t> split_feature, left_child, right_child;
    std::vector<uint32_t> threshold_bin;
    std::vector<uint8_t> default_left;
    std::vector<float> split_gain;
    std::vector<double> internal_value, internal_weight;
    std::vector<int64_t> internal_count;
    std::vector<double> leaf_value{0.0}, leaf_weight{0.0};
    std::vector<int64_t> leaf_count{0};
    std::vector<int32_t> leaf_parent{-1}, leaf_depth{0};
    std::vector<uint32_t> left_bins;  // [node][8]: the bins that go left

    // tree.rs:143-177
    uint32_t split(uint32_t leaf, int32_t feature, uint32_t threshold, bool dl, double lv, double rv, int64_t lc,
                   int64_t rc, double lw, double rw, float gain) {
        int32_t node = static_cast<int32_t>(num_leaves - 1);
        uint32_t new_leaf = num_leaves;
        int32_t parent = leaf_parent[leaf];
        if (parent >= 0) {
            if (left_child[parent] == ~static_cast<int32_t>(leaf)) left_child[parent] = node;
            else right_child[parent] = node;
        }
        split_feature.push_back(feature);
        split_gain.push_back(gain);
        threshold_bin.push_back(threshold);
        default_left.push_back(dl ? 1 : 0);
        left_child.push_back(~static_cast<int32_t>(leaf));
        right_child.push_back(~static_cast<int32_t>(new_leaf));
        internal_weight.push_back(leaf_weight[leaf]);
        internal_value.push_back(leaf_value[leaf]);
        internal_count.push_back(lc + rc);
        leaf_value[leaf] = nan_to_zero(lv);
        leaf_weight[leaf] = lw;
        leaf_count[leaf] = lc;
        leaf_value.push_back(nan_to_zero(rv));
        leaf_weight.push_back(rw);
        leaf_count.push_back(rc);
        leaf_parent[leaf] = node;
        leaf_parent.push_back(node);
        int32_t depth = leaf_depth[leaf] + 1;
        leaf_depth[leaf] = depth;
        leaf_depth.push_back(depth);
        ++num_leaves;
        return new_leaf;
    }
    void shrink(double rate) {  // tree.rs:180-185
        for (double &v : leaf_value) v = round_to_zero(v * rate);
        for (double &v : internal_value) v = round_to_zero(v * rate);
    }
    void add_bias(double bias) {  // tree.rs:188-193
        for (double &v : leaf_value) v = round_to_zero(v + bias);
        for (double &v : internal_value) v = round_to_zero(v + bias);
    }
};

// ---------------------------------------------------------------------------------------------------------
// The context
// ---------------------------------------------------------------------------------------------------------

constexpr uint32_t RANK_DEVICE_MAX = 512;  // rows of the largest query k_rank_pairs takes (longer ones: the host's)
constexpr uint32_t HIST_MIN_ROWS = 2048;   // rows per histogram workgroup before another one is used
constexpr uint64_t ROW_BLOCK = 256;

struct Slab {
    uint32_t width = 0;            // W: LDS and partial columns
    bool wide = false;             // two-byte bins: W / 4 features, each 4 virtual columns (k_hist<W, true>)
    uint32_t pack = 1;             // byte bins, `pack` features of at most 256 / pack bins a column (k_hist<W, false, pack>)
    bool q32 = false;              // separate 32-bit g and h LDS counters (k_hist<W, wide, 1, true>)
    uint32_t dense_passes = 0;     // a dense slab (k_hist<128, false, 1, false, DP>): features stacked by bin count
    uint32_t dense_row = 0;        // its row bytes (128 per feature a column)
    std::vector<uint32_t> pos_word, slot_flat;  // its tables (host): per row byte its LDS word, per slot its flat bin + 1
    uint64_t pos_off = 0, slot_off = 0;         // and their places in Context::slab_pos_word / slab_slot_flat
    std::vector<uint32_t> feats;   // feature ids
    uint64_t bins_off = 0;         // its rows in Context::slab_bins: [rows][row_bytes()]
    uint64_t col_bins_off = 0;     // its col_bins in Context::slab_col_bins (slots() entries)
    DevBuf<uint32_t> col_offset, col_bins, col_stride;  // per feature slot: segment * W + column (virtual column)
    uint32_t row_bytes() const { return dense_passes ? dense_row : (wide ? width / 2 : width * pack); }
    uint32_t capacity() const { return dense_passes ? dense_row : (wide ? width / 4 : width * pack); }
    uint32_t seg_shift() const { return pack == 4 ? 6u : (pack == 2 ? 7u : 8u); }
    uint32_t slots() const { return width * pack; }  // entries of the per-slot arrays
    uint32_t kernel() const {  // launch key
        return dense_passes ? 3000u + dense_passes : width + (wide ? 1u : 0u) + (pack > 1 ? pack : 0u) + (q32 ? 1000u : 0u);
    }
    bool same_launch(const Slab &o) const { return kernel() == o.kernel() && row_bytes() == o.row_bytes(); }
    uint64_t step_partial_off = 0;  // the slab's partials in the step partial buffer, in {g, h} pairs
};

// Where k_repack writes one feature's bins.
struct RepackTo {
    uint8_t *col;        // its column-major bins
    uint32_t col16;      // two bytes per bin there
    uint8_t *slab;       // its slab's rows (nullptr: none)
    uint32_t row_bytes;  // bytes per slab row
    uint32_t slab_wide;  // two bytes per bin in the slab row
    uint32_t slab_col;   // its byte (or two-byte) position in the slab row
    uint32_t num_bins;   // the feature's bins: a larger bin sets *bad
    uint32_t *bad;       // (nullptr: no check)
};

struct DevData {
    uint64_t rows = 0;
    DevBuf<uint8_t> col;  // [nt feature][rows], one byte per bin, or two (Context::col16)
    DevBuf<float> scores;
};

// Event timing of the histogram-building kernels and algorithmic byte counts (see srocm_profile_read).
struct Profile {
    bool on = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> hist_events, step_events, part_events;
    double hist_launches = 0, hist_ms = 0, hist_bytes = 0;  // k_hist: root and trait histograms
    double step_launches = 0, step_ms = 0, step_bytes = 0;  // k_step_rows: split steps
    double builds = 0, rows = 0, bins = 0, part_rows = 0;
    double part_launches = 0, part_ms = 0;                  // trait partitions
    double steps = 0, expansions = 0, splits = 0;           // device growth: split steps, leaves expanded, kept
    // the line model of the split steps' gathers (srocm_profile mode 2; k_sector_model): parent rows, their
    // split-bin lines, built rows, their gradient lines, split-bin lines shared over each step's jobs, partials
    // written, of those packed, and the sparse jobs' parent rows, split-bin lines and built rows
    bool sectors = false;
    DevBuf<unsigned long long> sector_counts;
    DevBuf<uint32_t> sector_bits;
    double sector[10] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    double rank_redos = 0;  // lambdarank gradients whose device factors were flagged and made again by the host
    std::vector<hipEvent_t> pool;
    void reset() {
        hist_launches = hist_ms = hist_bytes = step_launches = step_ms = step_bytes = 0;
        builds = rows = bins = part_rows = part_launches = part_ms = 0;
        steps = expansions = splits = 0;
        for (double &v : sector) v = 0;
        rank_redos = 0;
    }
};

struct GrowLeaf {
    srocm_leaf_range range{};
    double ug = 0.0, uh = 0.0;
    int64_t count = 0;
    int slot = -1;  // device histogram slot, -1: none
    std::vector<uint8_t> splittable;
    bool has_best = false;
    SplitOut best{};
};

struct Context {
    int device = 0;
    hipStream_t stream = nullptr;
    hipStream_t copy_stream = nullptr;  // a grown tree's readback, beside the kernels queued after the tree's steps
    std::string error;
    std::string device_name;
    uint32_t cus = 256;
    bool loaded = false;

    // layout
    uint32_t nf = 0;
    std::vector<srocm_feature> feats;
    uint64_t total_bins = 0;
    std::vector<std::vector<int32_t>> group_col_nt;
    std::vector<int32_t> feat_nt;
    std::vector<uint32_t> nt_feat;
    std::vector<Slab> slabs;
    uint64_t rows = 0, row_offset = 0;
    uint32_t max_width = 32;
    bool q32 = false;  // slabs laid out for separate 32-bit g and h LDS counters (set_mode)
    // every slab's rows in one buffer, each slab's at a multiple of 256 bytes, slabs of one row length
    // slab_stride() apart, so that a k_step_rows launch finds its later slabs by arithmetic
    DevBuf<uint8_t> slab_bins;
    DevBuf<uint32_t> slab_col_bins;  // every slab's col_bins, consecutive
    DevBuf<uint32_t> slab_pos_word, slab_slot_flat;  // the dense slabs' tables, consecutive
    uint32_t hist_cap = 0;     // k_hist workgroups a leaf is spread over at most
    uint32_t step_target = 0;  // k_step_rows workgroups a step is spread over (its grid: step_target + JMAX)
    uint32_t col16 = 0;                     // some group has two-byte bins: column-major bins are u16
    bool has_narrow = true, has_wide = false;  // features of one-byte / two-byte bins (a scan kernel each)
    std::vector<uint32_t> group_bits;  // per group: bits per bin, 8, 16 (wide slabs) or 4 (two to a byte)
    std::vector<uint32_t> nt_slab, nt_slab_col;  // per non-trivial feature: its slab and column there

    DevData train;
    std::vector<DevData> valid;
    DevBuf<float> label, weight, grad, hess;
    bool has_weight = false;
    std::vector<float> h_label_v, h_weight_v;
    DevBuf<int32_t> packed, partial;
    DevBuf<uint32_t> part, part2, block_left, scalars;
    DevBuf<uint32_t> maxima;  // the gradient maxima, MAX_SLOTS pairs
    bool maxima_clear = false; // maxima holds zeros on the stream (k_quant_spec cleared it after reading)
    DevBuf<uint8_t> codes0, codes1;  // grown trees: each row's gradient code beside its id in part / part2
    DevBuf<FeatDev> dfeats;
    DevBuf<ColGroup> d_cgs;
    DevBuf<uint32_t> d_fmt;  // per slab and k_step_rows workgroup: the format of its partial (1 packed, 0 pairs)
    DevBuf<int32_t> unit_feat;   // k_step_scan's units: UNIT_FEATS numerical features each, -1 padding
    DevBuf<uint32_t> unit_segl;  // and their lanes a feature (64, 16, 4)
    DevBuf<uint32_t> cat_feats;  // the categorical features of the slabs
    uint32_t ncat = 0;
    uint32_t ncg = 0;  // column groups of k_step_reduce
    uint32_t nsg = 0;  // scan units of k_step_scan
    bool has_seg_units = false;  // some units scan several features (k_step_scan_seg)
    uint32_t nseg_units = 0;     // those units, first in the unit list
    bool has_narrow64 = false;   // some units scan one byte feature (k_step_scan<false>)
    uint64_t step_partial_pairs = 0;
    uint32_t part_len = 0;
    std::vector<uint8_t> used;
    uint32_t objective = SROCM_OBJ_REGRESSION;
    double sigmoid = 1.0;
    int64_t max_gq = 1, max_hq = 1;  // the last quantization's largest |g| and h units
    bool quantized_once = false;

    Pinned<int64_t> h_hist;
    Pinned<uint32_t> h_u32;
    Pinned<uint8_t> h_result;
    Pinned<uint8_t> h_stage;  // per-split uploads (jobs, evaluate flags), rewritten only after a sync

    DevBuf<DevNode> d_nodes;
    Pinned<DevNode> h_nodes;
    Pinned<unsigned long long> h_sums;  // leaf sums on their way to the host
    DevBuf<double> d_leaf_vw;           // per tree of a boosting call (2 GROW_MAX_LEAVES + 1 each): its renewed leaf
                                        // values, then (from GROW_MAX_LEAVES) weights, then the gate
    DevBuf<uint32_t> d_gate;            // the boosted tree's leaves once it is complete with a split (k_tree_nodes)
    DevBuf<DevScales> d_scales;         // the boosting loop's quantization, made on the device (k_quant_spec)
    const DevScales *grow_dsc = nullptr;  // set while the boosting loop grows: the scales of GrowState
    hipEvent_t tree_event = nullptr;    // a grown tree's readback has landed
    hipEvent_t steps_event = nullptr;   // a batch of split steps has ended (the readback waits for it)
    Pinned<double> h_leaf_vw;           // and on the host, copied once at the end of the call
    Pinned<float> h_lv;
    DevBuf<uint16_t> leaf_of;  // each training row's leaf in the last tree (k_tree_leaves)
    DevBuf<float> d_leaf_values;
    DevBuf<LeafJob> d_leaf_jobs;
    DevBuf<unsigned long long> d_leaf_out;

    srocm_rank::Ranker ranker;  // lambdarank: the setup, the sigmoid and discount tables
    Pinned<float> h_rank_scores, h_rank_grad, h_rank_hess;
    // lambdarank: the queries of at most RANK_DEVICE_MAX rows run on the device (k_rank_pairs, one wave a query,
    // largest first so that the launch's tail is short), the longer ones on the host's threads. rank_nmax: the power
    // of two the device's queries fit (0: none); the setup, the tables and the per-row / per-query sums
    uint32_t rank_nmax = 0;
    std::vector<uint32_t> rank_dev_q, rank_host_q;  // the device's queries (largest first) and the host's
    DevBuf<uint32_t> d_rank_bounds, d_rank_queries;
    DevBuf<double> d_rank_imd, d_rank_gain, d_rank_table, d_rank_disc, d_rank_lam, d_rank_hes, d_rank_qsum, d_rank_factor;
    Pinned<double> h_rank_qsum, h_rank_factor;
    std::unique_ptr<srocm_rank::WorkPool> rank_pool;  // host threads for the factors and the host's queries
    hipEvent_t rank_event = nullptr;                   // the host's queries' scores have arrived
    // The device's factors (k_rank_scale, RANK_FACTOR_DEVICE): its flag that some query's could differ from the
    // host's comes back on the copy stream; while `rank_flag_pending`, the last gradients wait for that verdict
    // (rank_factors_vetoed). SROCM_TEST_RANK_FALLBACK=1 at load makes every query raise it (a test of the fallback).
    DevBuf<uint32_t> d_rank_flag;
    DevBuf<double> d_rank_pair;  // per query: the device's factors from both ends of the log2 bracket
    Pinned<uint32_t> h_rank_flag;
    hipEvent_t rank_flag_event = nullptr;
    bool rank_flag_pending = false, rank_flag_queued = false, rank_force_fallback = false;

    Profile prof;
    int2 *scratch_at = nullptr;  // this device's copy of `scratch` (srocm_histogram_noalloc)

    ~Context() {
        if (tree_event) (void)hipEventDestroy(tree_event);
        if (steps_event) (void)hipEventDestroy(steps_event);
        if (rank_event) (void)hipEventDestroy(rank_event);
        if (rank_flag_event) (void)hipEventDestroy(rank_flag_event);
        for (auto &e : prof.hist_events) {
            (void)hipEventDestroy(e.first);
            (void)hipEventDestroy(e.second);
        }
        for (auto &e : prof.part_events) {
            (void)hipEventDestroy(e.first);
            (void)hipEventDestroy(e.second);
        }
        for (auto &e : prof.step_events) {
            (void)hipEventDestroy(e.first);
            (void)hipEventDestroy(e.second);
        }
        for (auto e : prof.pool) (void)hipEventDestroy(e);
        if (copy_stream) (void)hipStreamDestroy(copy_stream);
        if (stream) (void)hipStreamDestroy(stream);
    }

    void sync() { hip_check(hipStreamSynchronize(stream), "stream synchronize"); }

    void require_loaded() const {
        if (!loaded) fail(SROCM_ERR_DEVICE, "rocm backend used before load");
    }

    hipEvent_t event() {
        if (!prof.pool.empty()) {
            hipEvent_t e = prof.pool.back();
            prof.pool.pop_back();
            return e;
        }
        hipEvent_t e;
        hip_check(hipEventCreate(&e), "hipEventCreate");
        return e;
    }

    // Whether the last gradients' device factors were flagged (some query's could differ from the host's): then the
    // gradients are made again with the host's factors. Waits for the flag's copy, not for the stream.
    bool rank_factors_vetoed() {
        if (!rank_flag_pending) return false;
        queue_rank_flag();
        hip_check(hipEventSynchronize(rank_flag_event), "event synchronize");
        rank_flag_pending = false;
        if (h_rank_flag.p[0] == 0u) return false;
        prof.rank_redos += 1;  // counted whether or not profiling is on
        return true;
    }

    // ------------------------------------------------------------------------------------------------
    // load (cpu.rs:707-746 checks; device layout)
    // ------------------------------------------------------------------------------------------------

    // ObjectiveSetup::LambdaRank (backend/mod.rs:62-71) and the training set's query boundaries, checked as silvic's
    // setup checks them (objective/mod.rs:34-62; lambdarank.rs:172-188 for the labels)
    void load_ranking(const srocm_dataset *t, const srocm_objective *obj) {
        const uint64_t nq = t->num_queries;
        if (!t->query_boundaries || nq == 0) fail(SROCM_ERR_DATA, "ranking tasks require query information");
        if (t->query_boundaries[0] != 0 || t->query_boundaries[nq] != t->num_rows)
            fail(SROCM_ERR_DATA, "query boundaries must run from 0 to the number of rows");
        for (uint64_t q = 0; q < nq; ++q)
            if (t->query_boundaries[q + 1] < t->query_boundaries[q]) fail(SROCM_ERR_DATA, "query boundaries must not decrease");
        if (!obj->label_gain || obj->num_label_gain == 0) fail(SROCM_ERR_CONFIG, "lambdarank needs label gains");
        for (uint64_t r = 0; r < t->num_rows; ++r) {
            const float l = t->label[r];  // Rust's saturating casts: a NaN label passes every check as label 0
            if (std::fabs(static_cast<double>(l) - static_cast<double>(srocm_rank::label_as_i32(l))) > K_EPS_H)
                fail(SROCM_ERR_DATA, "label should be int type (met " + std::to_string(l) + ") for ranking task");
            if (l < 0.0f) fail(SROCM_ERR_DATA, "label should be non-negative (met " + std::to_string(l) + ") for ranking task");
            if (srocm_rank::label_as_index(l) >= obj->num_label_gain)
                fail(SROCM_ERR_DATA, "label " + std::to_string(srocm_rank::label_as_index(l)) +
                                         " is not less than the number of label mappings (" + std::to_string(obj->num_label_gain) + ")");
        }
        srocm_rank::Setup st;
        st.sigmoid = obj->sigmoid;
        st.norm = obj->norm != 0;
        st.truncation_level = obj->truncation_level;
        st.label_gain.assign(obj->label_gain, obj->label_gain + obj->num_label_gain);
        if (obj->inverse_max_dcg) st.inverse_max_dcg.assign(obj->inverse_max_dcg, obj->inverse_max_dcg + nq);
        st.boundaries.assign(t->query_boundaries, t->query_boundaries + nq + 1);
        ranker.configure(std::move(st));
        if (!obj->inverse_max_dcg) ranker.derive_inverse_max_dcg(t->label);
    }

    // The split of the queries between the device (at most RANK_DEVICE_MAX rows, largest first) and the host, and the
    // device's copy of the lambdarank setup.
    void upload_ranking() {
        const srocm_rank::Setup &st = ranker.setup();
        const uint64_t nq = st.boundaries.size() - 1;
        rank_dev_q.clear();
        rank_host_q.clear();
        uint32_t biggest = 0;
        for (uint64_t q = 0; q < nq; ++q) {
            const uint32_t n = st.boundaries[q + 1] - st.boundaries[q];
            if (n > RANK_DEVICE_MAX) {
                rank_host_q.push_back(static_cast<uint32_t>(q));
            } else {
                rank_dev_q.push_back(static_cast<uint32_t>(q));
                biggest = std::max(biggest, n);
            }
        }
        std::stable_sort(rank_dev_q.begin(), rank_dev_q.end(), [&](uint32_t a, uint32_t b) {
            return st.boundaries[a + 1] - st.boundaries[a] > st.boundaries[b + 1] - st.boundaries[b];
        });
        if (!rank_pool) rank_pool = std::make_unique<srocm_rank::WorkPool>(std::max(1u, std::min(16u, std::thread::hardware_concurrency())));
        if (!rank_event) hip_check(hipEventCreateWithFlags(&rank_event, hipEventDisableTiming), "hipEventCreate");
        if (!rank_flag_event) hip_check(hipEventCreateWithFlags(&rank_flag_event, hipEventDisableTiming), "hipEventCreate");
        d_rank_flag.alloc(1);
        h_rank_flag.alloc(1);
        rank_flag_pending = false;
        const char *fb = std::getenv("SROCM_TEST_RANK_FALLBACK");
        rank_force_fallback = fb && fb[0] == '1';
        rank_nmax = 0;
        if (rank_dev_q.empty()) return;
        rank_nmax = 64;
        while (rank_nmax < biggest) rank_nmax <<= 1;
        d_rank_queries.alloc(rank_dev_q.size());
        hip_check(hipMemcpy(d_rank_queries.p, rank_dev_q.data(), rank_dev_q.size() * 4, hipMemcpyHostToDevice), "upload queries");
        d_rank_bounds.alloc(nq + 1);
        d_rank_imd.alloc(nq);
        d_rank_gain.alloc(st.label_gain.size());
        d_rank_table.alloc(srocm_rank::SIGMOID_BINS);
        d_rank_disc.alloc(srocm_rank::DISCOUNT_TABLE);
        d_rank_lam.alloc(std::max<uint64_t>(rows, 1));
        d_rank_hes.alloc(std::max<uint64_t>(rows, 1));
        d_rank_qsum.alloc(nq);
        d_rank_factor.alloc(nq);
        d_rank_pair.alloc(2 * static_cast<size_t>(nq));
        h_rank_qsum.alloc(nq);
        h_rank_factor.alloc(nq);
        hip_check(hipMemcpy(d_rank_bounds.p, st.boundaries.data(), (nq + 1) * 4, hipMemcpyHostToDevice), "upload queries");
        hip_check(hipMemcpy(d_rank_imd.p, st.inverse_max_dcg.data(), nq * 8, hipMemcpyHostToDevice), "upload max dcg");
        hip_check(hipMemcpy(d_rank_gain.p, st.label_gain.data(), st.label_gain.size() * 8, hipMemcpyHostToDevice), "upload gains");
        hip_check(hipMemcpy(d_rank_table.p, ranker.sigmoid_table().data(), srocm_rank::SIGMOID_BINS * 8, hipMemcpyHostToDevice),
                  "upload sigmoid table");
        hip_check(hipMemcpy(d_rank_disc.p, ranker.discounts().data(), srocm_rank::DISCOUNT_TABLE * 8, hipMemcpyHostToDevice),
                  "upload discounts");
    }

    // lambdarank gradients (lambdarank.rs:190-420). The device's queries: the pair sums (k_rank_pairs), then
    // k_rank_scale with the per-query normalization factors log2(1 + s) / s made on the device, whose flag comes back
    // on the copy stream (rank_factors_vetoed); with `host_factors` (the flag was raised), the factors are made on
    // the host's pool with the C library's log2 instead (the sums come back and the factors go out, so this waits for
    // the stream). The host's queries (more rows than k_rank_pairs takes): their scores come back first and their
    // gradients are computed on the pool (f64) while the device works on its own, then go out. The maxima are taken
    // on the device over every row.
    void ranking_gradients(bool host_factors) {
        const srocm_rank::Setup &st = ranker.setup();
        const uint32_t nq = static_cast<uint32_t>(st.boundaries.size() - 1);
        const uint32_t *qb = st.boundaries.data();
        const bool host = !rank_host_q.empty();
        // the host's queries' rows in few copies: query by query when they are few, else every row at once
        const bool by_query = rank_host_q.size() <= 64;
        auto each_host_range = [&](auto &&f) {
            if (!by_query) {
                f(0u, static_cast<uint32_t>(rows));
                return;
            }
            for (uint32_t q : rank_host_q) f(qb[q], qb[q + 1] - qb[q]);
        };
        if (host) {
            h_rank_scores.alloc(rows);
            h_rank_grad.alloc(rows);
            h_rank_hess.alloc(rows);
            each_host_range([&](uint32_t b, uint32_t n) {
                hip_check(hipMemcpyAsync(h_rank_scores.p + b, train.scores.p + b, static_cast<size_t>(n) * 4,
                                         hipMemcpyDeviceToHost, stream), "read scores");
            });
            hip_check(hipEventRecord(rank_event, stream), "event");
        }
        if (rank_nmax) {
            RankArgs ra{train.scores.p, label.p, d_rank_bounds.p, d_rank_imd.p, d_rank_gain.p, d_rank_table.p,
                        d_rank_disc.p, st.sigmoid, st.sigmoid * st.sigmoid, ranker.min_input(), ranker.max_input(),
                        ranker.idx_factor(), st.norm ? 1u : 0u, st.truncation_level, d_rank_lam.p, d_rank_hes.p,
                        d_rank_qsum.p, d_rank_queries.p, d_rank_flag.p};
            const uint32_t nd = static_cast<uint32_t>(rank_dev_q.size());
            switch (rank_nmax) {
            case 64: k_rank_pairs<64><<<nd, 64, 0, stream>>>(ra); break;
            case 128: k_rank_pairs<128><<<nd, 64, 0, stream>>>(ra); break;
            case 256: k_rank_pairs<256><<<nd, 64, 0, stream>>>(ra); break;
            default: k_rank_pairs<512><<<nd, 64, 0, stream>>>(ra); break;
            }
            launch_check("k_rank_pairs");
            if (st.norm && host_factors)
                hip_check(hipMemcpyAsync(h_rank_qsum.p, d_rank_qsum.p, static_cast<size_t>(nq) * 8, hipMemcpyDeviceToHost,
                                         stream), "read sums");
        }
        if (host) {  // while the device ranks its queries
            hip_check(hipEventSynchronize(rank_event), "event synchronize");
            ranker.gradients(rank_host_q.data(), rank_host_q.size(), h_rank_scores.p, h_label_v.data(),
                             has_weight ? h_weight_v.data() : nullptr, h_rank_grad.p, h_rank_hess.p, *rank_pool);
            each_host_range([&](uint32_t b, uint32_t n) {
                hip_check(hipMemcpyAsync(grad.p + b, h_rank_grad.p + b, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice,
                                         stream), "upload grad");
                hip_check(hipMemcpyAsync(hess.p + b, h_rank_hess.p + b, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice,
                                         stream), "upload hess");
            });
        }
        rank_flag_pending = false;
        if (rank_nmax) {
            const double *factor = nullptr;
            uint32_t mode = RANK_FACTOR_ONE;
            const uint32_t nd = static_cast<uint32_t>(rank_dev_q.size());
            if (st.norm && !host_factors) {
                mode = rank_force_fallback ? RANK_FACTOR_DEVICE_CHECKED : RANK_FACTOR_DEVICE;  // flag cleared by k_rank_pairs
                k_rank_factor<<<div_up(nd, 256), 256, 0, stream>>>(d_rank_queries.p, nd, d_rank_qsum.p, mode, d_rank_pair.p,
                                                                  d_rank_flag.p);
                launch_check("k_rank_factor");
            } else if (st.norm) {
                mode = RANK_FACTOR_HOST;
                sync();
                const uint32_t per = (nd + rank_pool->size() - 1) / rank_pool->size();
                rank_pool->run([&](unsigned w) {  // lambdarank.rs:287-300, as srocm_rank::Ranker takes it
                    for (uint32_t k = w * per; k < std::min(nd, (w + 1) * per); ++k) {
                        const uint32_t q = rank_dev_q[k];
                        h_rank_factor.p[q] = srocm_rank::norm_factor(true, h_rank_qsum.p[q]);
                    }
                });
                hip_check(hipMemcpyAsync(d_rank_factor.p, h_rank_factor.p, static_cast<size_t>(nq) * 8, hipMemcpyHostToDevice,
                                         stream), "upload factors");
                factor = d_rank_factor.p;
            }
            // the host's rows (uploaded above, from buffers that outlive the copies) are not written here
            k_rank_scale<<<static_cast<uint32_t>(rank_dev_q.size()), 64, 0, stream>>>(
                d_rank_bounds.p, d_rank_queries.p, d_rank_lam.p, d_rank_hes.p, factor, d_rank_pair.p, mode,
                has_weight ? weight.p : nullptr, grad.p, hess.p, d_rank_flag.p);
            launch_check("k_rank_scale");
            rank_flag_pending = mode >= RANK_FACTOR_DEVICE;
        }
        k_max_abs<<<grid_rows(rows), 256, 0, stream>>>(grad.p, hess.p, rows, maxima.p);
        launch_check("k_max_abs");
        rank_flag_queued = false;  // queue_rank_flag copies it, once the kernels after these are queued
    }

    // The device factors' flag, copied on the copy stream behind the kernels queued so far (the boosting loop calls
    // this once the iteration's quantization is queued, so the API calls leave no gap between its kernels).
    void queue_rank_flag() {
        if (!rank_flag_pending || rank_flag_queued) return;
        hip_check(hipEventRecord(rank_event, stream), "event");
        hip_check(hipStreamWaitEvent(copy_stream, rank_event, 0), "stream wait");
        hip_check(hipMemcpyAsync(h_rank_flag.p, d_rank_flag.p, 4, hipMemcpyDeviceToHost, copy_stream), "read rank flag");
        hip_check(hipEventRecord(rank_flag_event, copy_stream), "event");
        rank_flag_queued = true;
    }

    void load(const srocm_dataset *t, const srocm_dataset *const *v, uint32_t nv, const srocm_objective *obj) {
        if (!t || !obj) fail(SROCM_ERR_DATA, "load needs a training set and an objective");
        pending_order.on = false;
        if (t->num_rows > 0xFFFFFFFFull) fail(SROCM_ERR_UNSUPPORTED, std::to_string(t->num_rows) + " rows on one rank; the limit is 2^32 - 1");
        if (obj->kind == SROCM_OBJ_LAMBDARANK) {
            load_ranking(t, obj);
        } else if (obj->kind != SROCM_OBJ_REGRESSION && obj->kind != SROCM_OBJ_BINARY) {
            fail(SROCM_ERR_CONFIG, "unknown objective");
        }
        auto check_layout = [&](const srocm_dataset *d) {
            if (d->num_groups != t->num_groups || d->num_features != t->num_features)
                fail(SROCM_ERR_DATA, "validation set binned with a different layout than the training set");
            for (uint32_t g = 0; g < d->num_groups; ++g) {
                if (!d->groups[g].data && d->num_rows) fail(SROCM_ERR_DATA, "group without data");
                const uint32_t a = d->groups[g].bin_bits ? d->groups[g].bin_bits : 8u;
                const uint32_t b = t->groups[g].bin_bits ? t->groups[g].bin_bits : 8u;
                if (a != b || d->groups[g].row_stride != t->groups[g].row_stride)
                    fail(SROCM_ERR_DATA, "validation set binned with a different layout than the training set");
            }
        };
        for (uint32_t i = 0; i < nv; ++i) check_layout(v[i]);
        loaded = false;
        nf = t->num_features;
        feats.assign(t->features, t->features + nf);
        total_bins = t->total_bins;
        rows = t->num_rows;
        row_offset = t->row_offset;
        objective = obj->kind;
        sigmoid = obj->sigmoid;
        // feature checks (cpu.rs:178-223) and the column-major order of non-trivial features
        feat_nt.assign(nf, -1);
        nt_feat.clear();
        group_col_nt.assign(t->num_groups, {});
        group_bits.assign(t->num_groups, 8);
        col16 = 0;
        for (uint32_t g = 0; g < t->num_groups; ++g) {
            const uint32_t bits = t->groups[g].bin_bits == 0 ? 8u : t->groups[g].bin_bits;
            if (bits != 4 && bits != 8 && bits != 16)
                fail(SROCM_ERR_DATA, "group " + std::to_string(g) + " has " + std::to_string(bits) + "-bit bins");
            group_bits[g] = bits;
            group_col_nt[g].assign(static_cast<size_t>(t->groups[g].row_stride) * (bits == 4 ? 2 : 1), -1);
            if (bits == 16) col16 = 1;
        }
        uint64_t bins_seen = 0;
        for (uint32_t f = 0; f < nf; ++f) {
            const srocm_feature &m = feats[f];
            if (m.num_bins == 0) continue;
            if (m.kind != SROCM_BINS_NUMERICAL && m.kind != SROCM_BINS_CATEGORICAL) fail(SROCM_ERR_DATA, "bad feature kind");
            if (m.group >= t->num_groups) fail(SROCM_ERR_DATA, "feature in a missing group");
            const srocm_group &g = t->groups[m.group];
            const uint32_t bits = group_bits[m.group];
            if (bits == 8 && m.num_bins > 256) fail(SROCM_ERR_UNSUPPORTED, "a feature of one-byte bins has more than 256 bins");
            if (bits == 16 && (m.kind != SROCM_BINS_NUMERICAL || m.num_bins > 1024))
                fail(SROCM_ERR_UNSUPPORTED, "two-byte bins hold numerical features of at most 1024 bins");
            if (bits == 4 && m.num_bins > 16) fail(SROCM_ERR_UNSUPPORTED, "a feature of 4-bit bins has more than 16 bins");
            const uint64_t end_byte = bits == 4 ? m.column / 2 + 1 : m.column + bits / 8;  // past the feature's bytes
            if (end_byte > g.row_stride || m.hist_offset < g.hist_offset ||
                m.hist_offset - g.hist_offset + m.num_bins > g.total_bins || m.hist_offset + m.num_bins > total_bins)
                fail(SROCM_ERR_DATA, "feature " + std::to_string(f) + " lies outside its group's bins or row");
            feat_nt[f] = static_cast<int32_t>(nt_feat.size());
            group_col_nt[m.group][m.column] = feat_nt[f];
            nt_feat.push_back(f);
            bins_seen += m.num_bins;
        }
        (void)bins_seen;
        q32 = false;
        hist_cap = step_target = cus;
        build_slabs();
        // device buffers
        scalars.alloc(16);
        maxima.alloc(2 * MAX_SLOTS);
        maxima_clear = false;
        hip_check(hipMemsetAsync(scalars.p + 15, 0, 4, stream), "zero bin check");
        train = DevData{};
        upload_bins(t, train, true);
        valid.clear();
        for (uint32_t i = 0; i < nv; ++i) {
            DevData d;
            upload_bins(v[i], d, false);
            valid.push_back(std::move(d));
        }
        hip_check(hipMemcpyAsync(h_u32.p, scalars.p + 15, 4, hipMemcpyDeviceToHost, stream), "read bin check");
        sync();
        if (h_u32.p[0]) fail(SROCM_ERR_DATA, "a bin at or above its feature's num_bins");
        label.alloc(rows);
        h_label_v.assign(t->label, t->label + rows);
        hip_check(hipMemcpy(label.p, t->label, rows * sizeof(float), hipMemcpyHostToDevice), "upload label");
        has_weight = t->weight != nullptr;
        h_weight_v.clear();
        if (has_weight) {
            weight.alloc(rows);
            h_weight_v.assign(t->weight, t->weight + rows);
            hip_check(hipMemcpy(weight.p, t->weight, rows * sizeof(float), hipMemcpyHostToDevice), "upload weight");
        }
        if (obj->kind == SROCM_OBJ_LAMBDARANK) upload_ranking();
        grad.alloc(rows);
        hess.alloc(rows);
        packed.alloc(rows);
        part.alloc(rows);
        part2.alloc(rows);
        block_left.alloc(cus * 4 + 16);
        std::vector<FeatDev> fd(nf);
        has_narrow = has_wide = false;
        for (uint32_t f = 0; f < nf; ++f) {
            fd[f] = FeatDev{feats[f].num_bins, feats[f].hist_offset, feats[f].kind, feats[f].nan_bin,
                            feat_nt[f] < 0 ? 0u : static_cast<uint32_t>(feat_nt[f]),
                            feats[f].num_bins && group_bits[feats[f].group] == 16 ? 1u : 0u};
            // each feature's candidate (an empty one for a trivial feature) is written by the scan of its kind
            (fd[f].wide ? has_wide : has_narrow) = true;
        }
        dfeats.alloc(nf);
        hip_check(hipMemcpy(dfeats.p, fd.data(), nf * sizeof(FeatDev), hipMemcpyHostToDevice), "upload features");
        build_slab_tables();
        used.assign(nf, 1);
        part_len = 0;
        max_gq = max_hq = 1;
        quantized_once = false;
        grow_capacity = 0;
        pool.release();
        sync();
        loaded = true;
    }

    // Slabs. Two-byte features: up to 32 a slab, in feature order. Byte features: in the order of their bin classes
    // (more than 128 bins, more than 64, the rest; feature order within a class), up to 128 a slab while the slab
    // holds a feature of more than 128 bins, else up to 256. A slab's rows are the fewest bytes (32, 64, 128 or
    // 256) that hold its features, and its LDS columns hold as many features each (`pack`) as that row length and
    // its largest bin count allow: four of at most 64 bins, two of at most 128. With separate 32-bit g and h LDS
    // counters (q32) a slab has at most 64 columns and one feature a column: 64 byte or 16 two-byte features.
    void build_slabs() {
        slabs.clear();
        max_width = 32;
        nt_slab.assign(nt_feat.size(), 0);
        nt_slab_col.assign(nt_feat.size(), 0);
        {
            const uint32_t max_cols = q32 ? 64u : 128u;  // LDS columns a slab can take
            auto bin_class = [&](uint32_t i) {  // 4: at most 64 bins, 2: at most 128, 1: more
                const uint32_t nb = feats[nt_feat[i]].num_bins;
                return nb <= 64 ? 4u : (nb <= 128 ? 2u : 1u);
            };
            std::vector<uint32_t> narrow, wide;
            for (uint32_t c : {1u, 2u, 4u})
                for (uint32_t i = 0; i < nt_feat.size(); ++i)
                    if (group_bits[feats[nt_feat[i]].group] != 16 && bin_class(i) == c) narrow.push_back(i);
            for (uint32_t i = 0; i < nt_feat.size(); ++i)
                if (group_bits[feats[nt_feat[i]].group] == 16) wide.push_back(i);
            auto add_slab = [&](const std::vector<uint32_t> &members, size_t b, size_t e, bool is_wide) {
                Slab s;
                s.wide = is_wide;
                s.q32 = q32;
                uint32_t max_pack = q32 ? 1u : 4u;
                for (size_t k = b; k < e; ++k) {
                    nt_slab[members[k]] = static_cast<uint32_t>(slabs.size());
                    nt_slab_col[members[k]] = static_cast<uint32_t>(k - b);
                    s.feats.push_back(nt_feat[members[k]]);
                    max_pack = std::min(max_pack, bin_class(members[k]));
                }
                const uint32_t n = static_cast<uint32_t>(e - b);
                if (is_wide) {  // four virtual columns a feature
                    s.width = 4 * n <= 32 ? 32 : (4 * n <= 64 ? 64 : 128);
                } else {
                    uint32_t row = 32;
                    while (row < n) row *= 2;
                    s.pack = 1;
                    for (uint32_t p : {4u, 2u})
                        if (p <= max_pack && 32 * p <= row && row / p <= max_cols) {
                            s.pack = p;
                            break;
                        }
                    s.width = row / s.pack;
                }
                max_width = std::max(max_width, s.width);
                slabs.push_back(std::move(s));
            };
            for (size_t b = 0; b < narrow.size();) {
                const size_t per = std::min<size_t>(256, static_cast<size_t>(max_cols) * (q32 ? 1u : bin_class(narrow[b])));
                const size_t e = std::min(narrow.size(), b + per);
                add_slab(narrow, b, e, false);
                b = e;
            }
            for (size_t b = 0; b < wide.size(); b += max_cols / 4)
                add_slab(wide, b, std::min(wide.size(), b + max_cols / 4), true);
            // more than one slab of byte features: dense slabs instead, when they take fewer LDS columns
            size_t packed = 0;
            while (packed < slabs.size() && !slabs[packed].wide) ++packed;
            if (!q32 && packed > 1) build_dense(narrow, packed);
        }
    }

    // Dense slabs for the byte features `narrow` (non-trivial feature indices), in place of their `packed` slabs at
    // the start of `slabs`, when they take fewer LDS columns (so fewer partial words a workgroup) than those. The
    // features, largest bin count first, are dealt over k slabs in turn (k from the features' count and bins up,
    // until each slab fits); in a slab, each of the 128 LDS columns holds up to `per` features (per = ceil(its
    // features / 128)), stacked by bin count, a feature going to the column of fewest bins so far, whose bins must fit
    // its 256 rows. Feature j of column c is the row's byte c + 128 j. False (nothing changed) when they do not fit
    // or take no fewer columns.
    static constexpr uint32_t DENSE_FEATURES = 2048;  // a slab's features at most (rows of 2048 bytes, 8 passes)
    bool build_dense(const std::vector<uint32_t> &narrow, size_t packed) {
        uint32_t packed_cols = 0;
        for (size_t si = 0; si < packed; ++si) packed_cols += slabs[si].width;
        std::vector<uint32_t> order(narrow);
        std::stable_sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) {
            return feats[nt_feat[x]].num_bins > feats[nt_feat[y]].num_bins;
        });
        uint64_t total_bins = 0;
        for (uint32_t i : order) total_bins += feats[nt_feat[i]].num_bins;
        const size_t k0 = std::max<size_t>((order.size() + DENSE_FEATURES - 1) / DENSE_FEATURES, (total_bins + 32767) / 32768);
        for (size_t k = k0; k * 128 < packed_cols; ++k) {
            std::vector<Slab> out(k);
            std::vector<std::pair<uint32_t, uint32_t>> place(nt_feat.size());  // nt -> (slab, byte)
            bool ok = true;
            for (size_t si = 0; si < k && ok; ++si) {
                std::vector<uint32_t> part;
                for (size_t j = si; j < order.size(); j += k) part.push_back(order[j]);
                const uint32_t per = static_cast<uint32_t>((part.size() + 127) / 128);
                if (per * 128 > DENSE_FEATURES) {
                    ok = false;
                    break;
                }
                std::vector<uint32_t> sum(128, 0);
                std::vector<std::vector<uint32_t>> col(128);
                for (uint32_t i : part) {
                    const uint32_t nb = feats[nt_feat[i]].num_bins;
                    int best = -1;
                    for (int c = 0; c < 128; ++c)
                        if (col[c].size() < per && (best < 0 || sum[c] < sum[best])) best = c;
                    if (best < 0 || sum[best] + nb > 256) {
                        ok = false;
                        break;
                    }
                    col[best].push_back(i);
                    sum[best] += nb;
                }
                if (!ok) break;
                Slab &s = out[si];
                s.width = 128;
                s.dense_row = 128 * per;
                s.dense_passes = per <= 8 ? 4 : 8;  // 32 * per dwords a row, 64 a pass
                s.pos_word.resize(256ull * s.dense_passes);
                for (uint32_t p = 0; p < s.pos_word.size(); ++p) s.pos_word[p] = 256u * 128u + p % 128;  // the spare row
                s.slot_flat.assign(256ull * 128, 0u);
                for (uint32_t c = 0; c < 128; ++c) {
                    uint32_t base = 0;
                    for (uint32_t j = 0; j < col[c].size(); ++j) {
                        const uint32_t i = col[c][j], pos = c + 128 * j;
                        const srocm_feature &m = feats[nt_feat[i]];
                        s.pos_word[pos] = base * 128 + c;
                        for (uint32_t b = 0; b < m.num_bins; ++b) s.slot_flat[(base + b) * 128 + c] = m.hist_offset + b + 1;
                        place[i] = {static_cast<uint32_t>(si), pos};
                        base += m.num_bins;
                    }
                }
                for (uint32_t i : part) s.feats.push_back(nt_feat[i]);
                std::sort(s.feats.begin(), s.feats.end());
            }
            if (!ok) continue;
            // the dense slabs replace the packed ones at the start of `slabs`
            slabs.erase(slabs.begin(), slabs.begin() + static_cast<std::ptrdiff_t>(packed));
            const uint32_t shift = static_cast<uint32_t>(k) - static_cast<uint32_t>(packed);  // later slabs move by this
            for (uint32_t i = 0; i < nt_feat.size(); ++i)
                if (group_bits[feats[nt_feat[i]].group] != 16) {
                    nt_slab[i] = place[i].first;
                    nt_slab_col[i] = place[i].second;
                } else {
                    nt_slab[i] += shift;
                }
            slabs.insert(slabs.begin(), std::make_move_iterator(out.begin()), std::make_move_iterator(out.end()));
            max_width = 32;
            for (auto &sl : slabs) max_width = std::max(max_width, sl.width);
            return true;
        }
        return false;
    }

    // The slab tables: per slab slot its feature's flat bins, the column groups of k_step_reduce, the numerical
    // features (in groups of CG_COLS) of k_step_scan, the categorical ones of k_step_cat, and the partial buffers.
    void build_slab_tables() {
        partial.alloc(static_cast<size_t>(hist_cap) * 256 * max_width * 2);
        std::vector<uint32_t> all_bins;  // slab_col_bins
        std::vector<uint32_t> all_pos, all_slot;  // slab_pos_word, slab_slot_flat
        for (auto &s : slabs) {
            // slot i: a byte feature's (column i % W, segment i / W); in a wide slab, virtual column i, bins
            // congruent to i / (W/4) mod 4 of feature i % (W/4); a dense slab's slots are in its own tables
            const uint32_t ns = s.slots();
            std::vector<uint32_t> off(ns, 0), nb(ns, 0), st(ns, 1);
            if (s.dense_passes) {
                s.pos_off = all_pos.size();
                all_pos.insert(all_pos.end(), s.pos_word.begin(), s.pos_word.end());
                s.slot_off = all_slot.size();
                all_slot.insert(all_slot.end(), s.slot_flat.begin(), s.slot_flat.end());
            }
            for (size_t c = 0; c < s.feats.size() && !s.dense_passes; ++c) {
                const srocm_feature &m = feats[s.feats[c]];
                if (!s.wide) {
                    off[c] = m.hist_offset;
                    nb[c] = m.num_bins;
                    continue;
                }
                for (uint32_t q = 0; q < 4; ++q) {
                    const size_t v = q * (s.width / 4) + c;
                    off[v] = m.hist_offset + q;
                    nb[v] = m.num_bins > q ? (m.num_bins - q + 3) / 4 : 0u;
                    st[v] = 4;
                }
            }
            s.col_offset.alloc(ns);
            s.col_bins.alloc(ns);
            s.col_stride.alloc(ns);
            hip_check(hipMemcpy(s.col_stride.p, st.data(), ns * 4, hipMemcpyHostToDevice), "upload slab");
            hip_check(hipMemcpy(s.col_offset.p, off.data(), ns * 4, hipMemcpyHostToDevice), "upload slab");
            hip_check(hipMemcpy(s.col_bins.p, nb.data(), ns * 4, hipMemcpyHostToDevice), "upload slab");
            s.col_bins_off = all_bins.size();
            all_bins.insert(all_bins.end(), nb.begin(), nb.end());
        }
        slab_col_bins.alloc(std::max<size_t>(all_bins.size(), 1));
        if (!all_bins.empty())
            hip_check(hipMemcpy(slab_col_bins.p, all_bins.data(), all_bins.size() * 4, hipMemcpyHostToDevice), "upload slab");
        slab_pos_word.alloc(std::max<size_t>(all_pos.size(), 1));
        slab_slot_flat.alloc(std::max<size_t>(all_slot.size(), 4));
        if (!all_pos.empty()) {
            hip_check(hipMemcpy(slab_pos_word.p, all_pos.data(), all_pos.size() * 4, hipMemcpyHostToDevice), "upload dense slab");
            hip_check(hipMemcpy(slab_slot_flat.p, all_slot.data(), all_slot.size() * 4, hipMemcpyHostToDevice), "upload dense slab");
        }
        // groups of CG_COLS slab columns for k_step_reduce, the numerical features in groups of CG_COLS for
        // k_step_scan, and the categorical ones for k_step_cat
        {
            std::vector<ColGroup> cg;
            std::vector<int32_t> sfeat;
            std::vector<uint32_t> cats;
            uint64_t poff = 0;
            for (size_t si = 0; si < slabs.size(); ++si) {
                Slab &s = slabs[si];
                s.step_partial_off = poff;
                // a wide slab's virtual column v holds bins q, q + 4, ... (q = v / (W/4)) of feature v % (W/4); a
                // packed slab's column c holds feature seg * W + c in bins [seg, seg + 1) * 2^seg_shift
                const uint32_t cap = s.capacity();
                for (uint32_t c0 = 0; c0 < s.width; c0 += CG_COLS) {
                    ColGroup x{poff, s.width, c0, static_cast<uint32_t>(si) * k1_groups(), {}, {}, {}, s.seg_shift(),
                               s.dense_passes ? 1u : 0u, static_cast<uint32_t>(s.slot_off)};
                    for (uint32_t k = 0; k < CG_COLS && !s.dense_passes; ++k) {
                        const uint32_t v = c0 + k;
                        x.stride[k] = s.wide ? 4u : 1u;
                        for (uint32_t seg = 0; seg < s.pack; ++seg) {
                            const uint32_t c = s.wide ? v % cap : seg * s.width + v, q = s.wide ? v / cap : 0u;
                            const bool real = c < s.feats.size();
                            const srocm_feature &m = feats[real ? s.feats[c] : 0];
                            x.offset[seg][k] = real ? m.hist_offset + q : 0u;
                            x.bins[seg][k] = real && m.num_bins > q ? (m.num_bins - q + (s.wide ? 3 : 0)) / (s.wide ? 4 : 1) : 0u;
                        }
                    }
                    cg.push_back(x);
                }
                for (uint32_t f : s.feats) {
                    if (feats[f].kind == SROCM_BINS_CATEGORICAL) cats.push_back(f);
                    else sfeat.push_back(static_cast<int32_t>(f));
                }
                poff += static_cast<uint64_t>(k1_groups()) * step_partial_stride(s.width);
            }
            // scan units: byte features of at most 16 bins 16 a wave, of at most 64 bins 4 a wave, the others (and
            // two-byte features) one a wave; when that saves under a quarter of the waves, every feature one a wave
            // (the units of several features take a kernel of their own)
            auto unit_lanes = [&](int32_t f) {
                const uint32_t nb = feats[f].num_bins;
                return group_bits[feats[f].group] == 16 || nb > 64 ? 64u : (nb > 16 ? 16u : 4u);
            };
            size_t seg_units = 0;
            for (uint32_t segl : {4u, 16u, 64u}) {
                size_t n = 0;
                for (int32_t f : sfeat) n += unit_lanes(f) == segl;
                seg_units += (n + 64 / segl - 1) / (64 / segl);
            }
            const bool segmented = seg_units * 4 <= sfeat.size() * 3;
            std::vector<int32_t> ufeat;
            std::vector<uint32_t> usegl;
            for (uint32_t segl : {4u, 16u, 64u}) {
                std::vector<int32_t> members;
                for (int32_t f : sfeat)
                    if ((segmented ? unit_lanes(f) : 64u) == segl) members.push_back(f);
                const size_t per = 64 / segl;
                for (size_t b = 0; b < members.size(); b += per) {
                    for (size_t k = 0; k < UNIT_FEATS; ++k)
                        ufeat.push_back(k < per && b + k < members.size() ? members[b + k] : -1);
                    usegl.push_back(segl);
                }
            }
            d_fmt.alloc(std::max<size_t>(slabs.size(), 1) * k1_groups());
            ncg = static_cast<uint32_t>(cg.size());
            nsg = static_cast<uint32_t>(usegl.size());
            has_seg_units = segmented;
            nseg_units = 0;
            while (nseg_units < usegl.size() && usegl[nseg_units] != 64) ++nseg_units;
            has_narrow64 = false;
            for (size_t u = 0; u < usegl.size(); ++u)
                if (usegl[u] == 64 && group_bits[feats[ufeat[u * UNIT_FEATS]].group] != 16) has_narrow64 = true;
            step_partial_pairs = std::max<uint64_t>(poff, 1);
            d_cgs.alloc(std::max<size_t>(cg.size(), 1));
            unit_feat.alloc(std::max<size_t>(ufeat.size(), 1));
            unit_segl.alloc(std::max<size_t>(usegl.size(), 1));
            if (!cg.empty())
                hip_check(hipMemcpy(d_cgs.p, cg.data(), cg.size() * sizeof(ColGroup), hipMemcpyHostToDevice), "upload column groups");
            if (!ufeat.empty()) {
                hip_check(hipMemcpy(unit_feat.p, ufeat.data(), ufeat.size() * 4, hipMemcpyHostToDevice), "upload scan units");
                hip_check(hipMemcpy(unit_segl.p, usegl.data(), usegl.size() * 4, hipMemcpyHostToDevice), "upload scan units");
            }
            ncat = static_cast<uint32_t>(cats.size());
            cat_feats.alloc(std::max<size_t>(cats.size(), 1));
            if (!cats.empty())
                hip_check(hipMemcpy(cat_feats.p, cats.data(), cats.size() * 4, hipMemcpyHostToDevice), "upload categorical features");
        }
    }

    // Chooses between packed 16/16 LDS words and separate 32-bit g and h counters (`q32`, for quantized units the
    // packed words would flush every few rows), and the workgroup counts: with units of up to `units`, no
    // workgroup may add up more than (2^31 - 1) / units rows, since its sums are 32-bit. Packed words take at most
    // 255 units, so one workgroup per compute unit always fits; separate counters take up to 65535, for which the
    // histogram and split-step workgroups are multiplied as the rows need. When the mode changes the slabs are laid
    // out again and refilled on the device from the column-major bins; when the counts change, the tables and
    // partial buffers follow.
    struct WorkgroupCounts {
        uint32_t hist_cap, step_target;  // k_hist workgroups at most, k_step_rows workgroups a step is spread over
    };
    WorkgroupCounts mode_counts(bool want, int64_t units) const {
        uint32_t hc = cus, st = cus;
        if (want) {
            const uint64_t cap = 2147483647ull / static_cast<uint64_t>(std::max<int64_t>(units, 1));  // rows a workgroup takes
            const uint64_t n = std::max<uint64_t>(rows, 1);
            // k_hist: div_up(n, groups) rows, rounded up to 64, at least HIST_MIN_ROWS (max_workgroup_rows)
            hc = static_cast<uint32_t>(std::max<uint64_t>(cus, div_up(n, cap - 128)));
            // k_step_rows: at most div_up(tiles + JMAX, target - JMAX) tiles of STEP_TILE rows
            st = static_cast<uint32_t>(std::max<uint64_t>(cus, div_up(div_up(n, STEP_TILE) + JMAX, cap / STEP_TILE) + JMAX));
        }
        return {hc, st};
    }
    void set_mode(bool want, int64_t units) {
        const WorkgroupCounts wc = mode_counts(want, units);
        const uint32_t hc = wc.hist_cap, st = wc.step_target;
        if (want == q32 && hc == hist_cap && st == step_target) return;
        sync();
        const bool relayout = want != q32;
        q32 = want;
        hist_cap = hc;
        step_target = st;
        if (!relayout) {
            build_slab_tables();
            if (grow_capacity) step_partial.alloc(2 * step_partial_pairs);
            sync();
            return;
        }
        build_slabs();
        alloc_slab_bins(rows);
        const uint64_t cb = col16 ? 2 : 1;
        for (uint32_t nt = 0; rows && nt < nt_feat.size(); ++nt) {
            const Slab &sl = slabs[nt_slab[nt]];
            RepackTo to{nullptr, col16, slab_bins.p + sl.bins_off, sl.row_bytes(), sl.wide ? 1u : 0u, nt_slab_col[nt], 0u, nullptr};
            repack(train.col.p + static_cast<size_t>(nt) * rows * cb, static_cast<uint32_t>(cb), 0, col16 ? 16u : 8u, rows, to);
        }
        build_slab_tables();
        if (grow_capacity) step_partial.alloc(2 * step_partial_pairs);
        sync();
    }

    // packed 16/16 words flush every fewer rows than this: separate counters instead
    static constexpr uint32_t Q32_BELOW_FLUSH = 256;
    static uint32_t packed_flush_rows(int64_t gq, int64_t hq) {
        return static_cast<uint32_t>(std::min(32767 / std::max<int64_t>(gq, 1), 65535 / std::max<int64_t>(hq, 1)));
    }

    // bytes from one slab's rows to the next slab's of the same row length
    uint64_t slab_stride(const Slab &sl) const { return (std::max<uint64_t>(rows, 1) * sl.row_bytes() + 255) & ~uint64_t(255); }

    // slab_bins for `n` rows (zeroed: padding bytes are bin 0), each slab at its offset
    void alloc_slab_bins(uint64_t n) {
        uint64_t total = 0;
        for (auto &sl : slabs) {
            sl.bins_off = total;
            total += (std::max<uint64_t>(n, 1) * sl.row_bytes() + 255) & ~uint64_t(255);
        }
        slab_bins.alloc(std::max<uint64_t>(total, 1));
        hip_check(hipMemsetAsync(slab_bins.p, 0, std::max<uint64_t>(total, 1), stream), "zero slabs");
    }

    // Repacks a dataset's groups into slab rows (training set) and column-major bins, on the device.
    void upload_bins(const srocm_dataset *d, DevData &out, bool with_slabs) {
        out.rows = d->num_rows;
        uint64_t n = d->num_rows;
        const uint64_t cb = col16 ? 2 : 1;
        out.col.alloc(std::max<uint64_t>(1, nt_feat.size() * n * cb));
        out.scores.alloc(std::max<uint64_t>(n, 1));
        hip_check(hipMemsetAsync(out.scores.p, 0, std::max<uint64_t>(n, 1) * sizeof(float), stream), "zero scores");
        if (with_slabs) alloc_slab_bins(n);
        if (n == 0) return;
        DevBuf<uint8_t> staging;
        for (uint32_t g = 0; g < d->num_groups; ++g) {
            const srocm_group &grp = d->groups[g];
            uint64_t bytes = n * grp.row_stride;
            staging.alloc(bytes);
            hip_check(hipMemcpyAsync(staging.p, grp.data, bytes, hipMemcpyHostToDevice, stream), "upload group");
            for (uint32_t c = 0; c < group_col_nt[g].size(); ++c) {
                int32_t nt = group_col_nt[g][c];
                if (nt < 0) continue;
                // every bin must be below its feature's count: the slabs' LDS addresses rely on it (checked after)
                RepackTo to{out.col.p + static_cast<size_t>(nt) * n * cb, col16, nullptr, 0, 0, 0,
                            feats[nt_feat[nt]].num_bins, scalars.p + 15};
                if (with_slabs) {
                    const Slab &sl = slabs[nt_slab[nt]];
                    to.slab = slab_bins.p + sl.bins_off;
                    to.row_bytes = sl.row_bytes();
                    to.slab_wide = sl.wide ? 1u : 0u;
                    to.slab_col = nt_slab_col[nt];
                }
                repack(staging.p, grp.row_stride, c, group_bits[g], n, to);
            }
            sync();  // staging is reused
        }
    }

    void repack(const uint8_t *src, uint32_t stride, uint32_t column, uint32_t bits, uint64_t n, const RepackTo &to);

    // ------------------------------------------------------------------------------------------------
    // gradients, quantization, partition reset
    // ------------------------------------------------------------------------------------------------

    std::pair<double, double> read_maxima() {
        hip_check(hipMemcpyAsync(h_u32.p, maxima.p, 8 * MAX_SLOTS, hipMemcpyDeviceToHost, stream), "read maxima");
        sync();
        uint32_t ug = 0, uh = 0;
        for (uint32_t k = 0; k < MAX_SLOTS; ++k) {
            ug = std::max(ug, h_u32.p[2 * k]);
            uh = std::max(uh, h_u32.p[2 * k + 1]);
        }
        float g, h;
        std::memcpy(&g, &ug, 4);
        std::memcpy(&h, &uh, 4);
        return {static_cast<double>(g), static_cast<double>(h)};
    }

    uint32_t grid_rows(uint64_t n) const { return static_cast<uint32_t>(std::min<uint64_t>(std::max<uint64_t>(div_up(n, 256), 1), cus * 8ull)); }

    std::pair<double, double> compute_gradients();
    void launch_gradients(bool host_factors);  // the gradients and their maxima, without waiting for them

    std::pair<double, double> set_gradients(const float *g, const float *h, uint64_t n) {
        require_loaded();
        if (n != rows) fail(SROCM_ERR_DEVICE, "gradient arrays of " + std::to_string(n) + " rows, expected " + std::to_string(rows));
        hip_check(hipMemcpyAsync(grad.p, g, n * 4, hipMemcpyHostToDevice, stream), "upload grad");
        hip_check(hipMemcpyAsync(hess.p, h, n * 4, hipMemcpyHostToDevice, stream), "upload hess");
        hip_check(hipMemsetAsync(maxima.p, 0, 8 * MAX_SLOTS, stream), "zero maxima");
        maxima_clear = false;
        k_max_abs<<<grid_rows(n), 256, 0, stream>>>(grad.p, hess.p, n, maxima.p);
        launch_check("k_max_abs");
        return read_maxima();
    }

    // The most rows one histogram workgroup adds up: k_hist spreads a leaf over at most hist_cap workgroups in
    // multiples of 64 rows (at least HIST_MIN_ROWS each); a split step gives a workgroup at most
    // ceil(tiles / (step_target - JMAX)) tiles of a job, the step's tiles being at most rows / STEP_TILE + JMAX.
    uint64_t max_workgroup_rows(const WorkgroupCounts &wc) const {
        const uint64_t n = std::max<uint64_t>(rows, 1);
        const uint64_t hist = div_up(std::max<uint64_t>(div_up(n, wc.hist_cap), HIST_MIN_ROWS), 64) * 64 + 64;
        const uint64_t share = wc.step_target > JMAX ? wc.step_target - JMAX : 1;
        const uint64_t step = div_up(div_up(n, STEP_TILE) + JMAX, share) * STEP_TILE;
        return std::max(hist, step);
    }

    // Quantized units a histogram can take: a packed word holds g as a signed 16-bit half and h as an unsigned one,
    // and a workgroup's sums of either are i32 (the reference's CPU sums are i64, cpu.rs:517-525), so
    // max_q * max_workgroup_rows() must stay below 2^31. Checked against the workgroup counts the mode for these
    // units takes, before set_mode changes anything, so a refused quantization leaves the context as it was.
    static void check_unit_range(int64_t grad_max_q, int64_t hess_max_q) {
        if (grad_max_q < 1 || grad_max_q > 32767 || hess_max_q < 1 || hess_max_q > 65535)
            fail(SROCM_ERR_UNSUPPORTED, "quantized units must lie in 1..=32767 for gradients and 1..=65535 for hessians");
    }
    bool q32_for(int64_t grad_max_q, int64_t hess_max_q) const {
        return packed_flush_rows(grad_max_q, hess_max_q) < Q32_BELOW_FLUSH;
    }
    void check_quant_units(int64_t grad_max_q, int64_t hess_max_q) const {
        check_unit_range(grad_max_q, hess_max_q);
        const uint64_t wg = max_workgroup_rows(mode_counts(q32_for(grad_max_q, hess_max_q), std::max(grad_max_q, hess_max_q)));
        if (static_cast<uint64_t>(std::max(grad_max_q, hess_max_q)) * wg > 2147483647ull)
            fail(SROCM_ERR_UNSUPPORTED, "quantized units up to " + std::to_string(std::max(grad_max_q, hess_max_q)) + " over " +
                                            std::to_string(wg) + " rows per histogram workgroup could overflow its 32-bit sums");
    }

    void quantize(const srocm_quant_spec &s) {
        require_loaded();
        check_quant_units(s.grad_max_q, s.hess_max_q);
        set_mode(q32_for(s.grad_max_q, s.hess_max_q), std::max(s.grad_max_q, s.hess_max_q));
        QuantDev q{s.inv_grad_scale, s.inv_hess_scale, s.grad_max_q, s.hess_max_q, s.constant_hessian, s.stochastic, s.seed, s.iteration};
        if (rows) {
            k_quantize<<<grid_rows(rows), 256, 0, stream>>>(grad.p, hess.p, packed.p, rows, row_offset, q);
            launch_check("k_quantize");
        }
        max_gq = s.grad_max_q;
        max_hq = s.hess_max_q;
        quantized_once = true;
    }

    uint32_t reset_partition(const srocm_bag &bag) {
        require_loaded();
        pending_order.on = false;  // the partition is rewritten
        if (rows == 0) {
            part_len = 0;
            return 0;
        }
        k_iota<<<grid_rows(rows), 256, 0, stream>>>(part.p, rows);
        launch_check("k_iota");
        if (bag.kind == SROCM_BAG_ALL) {
            part_len = static_cast<uint32_t>(rows);
            return part_len;
        }
        if (bag.kind != SROCM_BAG_BERNOULLI) fail(SROCM_ERR_CONFIG, "unknown bag kind");
        // a stable compaction: the in-bag rows, ascending (cpu.rs:816-823)
        PartArgs a = part_args(0, static_cast<uint32_t>(rows));
        a.col = nullptr;
        a.bag_seed = bag.seed;
        a.bag_round = bag.round;
        a.row_offset = row_offset;
        a.fraction = bag.fraction;
        run_partition(a, static_cast<uint32_t>(rows));
        hip_check(hipMemcpyAsync(h_u32.p, scalars.p, 4, hipMemcpyDeviceToHost, stream), "read bag count");
        sync();
        part_len = h_u32.p[0];
        return part_len;
    }

    // ------------------------------------------------------------------------------------------------
    // histograms
    // ------------------------------------------------------------------------------------------------

    // rows a packed word takes before its sums could leave their halves: g (low 16 bits, signed) within +-32767,
    // h (high 16 bits, never negative) at most 65535; with separate counters, rows before an i32 counter could
    // overflow (check_quant_units keeps a workgroup's rows below that)
    uint32_t flush_rows() const {
        if (q32) return static_cast<uint32_t>(2147483647 / std::max<int64_t>(std::max(max_gq, max_hq), 1));
        return packed_flush_rows(max_gq, max_hq);
    }

    uint32_t hist_groups(uint64_t n) const {
        uint32_t want = div_up(std::max<uint64_t>(n, 1), HIST_MIN_ROWS);
        return std::max<uint32_t>(1, std::min<uint32_t>(want, hist_cap));
    }

    // The histogram of rows part[begin..+count] (or the `side` child of that range split at *dev_left) into
    // `out` (i64 {g,h} per bin), and parent -= out when `parent` is set.
    // The features a histogram build evaluates: their columns, their bin bytes a row (two for a feature of
    // two-byte bins) and their bins (for the algorithmic byte counts of srocm_profile).
    struct HistUse {
        uint64_t columns = 0, bin_bytes = 0, bins = 0;
    };
    template <class Keep>
    HistUse hist_use(Keep &&keep) const {
        HistUse u;
        for (uint32_t f = 0; f < nf; ++f)
            if (keep(f) && feats[f].num_bins) {
                ++u.columns;
                u.bin_bytes += group_bits[feats[f].group] == 16 ? 2u : 1u;
                u.bins += feats[f].num_bins;
            }
        return u;
    }

    void launch_hist(uint32_t begin, uint32_t count, const uint32_t *dev_left, uint32_t side, int64_t *out,
                     int64_t *parent, const HistUse &use) {
        launch_hist_into(begin, count, dev_left, side, out, parent, use, partial.p, hist_groups(count), prof.on);
    }

    // launch_hist with the partials in `partials` (grid * 256 * max_width {g, h} pairs) over `grid` workgroups
    void launch_hist_into(uint32_t begin, uint32_t count, const uint32_t *dev_left, uint32_t side, int64_t *out,
                          int64_t *parent, const HistUse &use, int32_t *partials, uint32_t grid, bool profiled) {
        for (auto &s : slabs) {
            HistArgs a{slab_bins.p + s.bins_off, part.p, packed.p, partials, dev_left, begin, count, side, flush_rows(), grid, HIST_MIN_ROWS,
                       slab_pos_word.p + s.pos_off, s.row_bytes() / 4};
            hipEvent_t e0 = nullptr, e1 = nullptr;
            if (profiled) {
                e0 = event();
                e1 = event();
                hip_check(hipEventRecord(e0, stream), "event");
            }
            switch (s.kernel()) {
            case 32: k_hist<32><<<grid, 1024, 0, stream>>>(a); break;
            case 64: k_hist<64><<<grid, 1024, 0, stream>>>(a); break;
            case 128: k_hist<128><<<grid, 1024, 0, stream>>>(a); break;
            case 33: k_hist<32, true><<<grid, 1024, 0, stream>>>(a); break;
            case 65: k_hist<64, true><<<grid, 1024, 0, stream>>>(a); break;
            case 129: k_hist<128, true><<<grid, 1024, 0, stream>>>(a); break;
            case 36: k_hist<32, false, 4><<<grid, 1024, 0, stream>>>(a); break;
            case 68: k_hist<64, false, 4><<<grid, 1024, 0, stream>>>(a); break;
            case 34: k_hist<32, false, 2><<<grid, 1024, 0, stream>>>(a); break;
            case 66: k_hist<64, false, 2><<<grid, 1024, 0, stream>>>(a); break;
            case 130: k_hist<128, false, 2><<<grid, 1024, 0, stream>>>(a); break;
            case 3004: k_hist<128, false, 1, false, 4><<<grid, 1024, 0, stream>>>(a); break;
            case 3008: k_hist<128, false, 1, false, 8><<<grid, 1024, 0, stream>>>(a); break;
            case 1032: k_hist<32, false, 1, true><<<grid, 1024, 0, stream>>>(a); break;
            case 1064: k_hist<64, false, 1, true><<<grid, 1024, 0, stream>>>(a); break;
            case 1033: k_hist<32, true, 1, true><<<grid, 1024, 0, stream>>>(a); break;
            case 1065: k_hist<64, true, 1, true><<<grid, 1024, 0, stream>>>(a); break;
            default: throw std::logic_error("no histogram kernel for the slab");
            }
            launch_check("k_hist");
            if (profiled) {
                hip_check(hipEventRecord(e1, stream), "event");
                prof.hist_events.emplace_back(e0, e1);
                prof.hist_launches += 1;
            }
            ReduceArgs r{partials, s.col_offset.p, s.col_bins.p, s.col_stride.p, out, parent, dev_left, begin, count, side, grid, HIST_MIN_ROWS, s.width, s.seg_shift(),
                         s.dense_passes ? slab_slot_flat.p + s.slot_off : nullptr};
            k_hist_reduce<<<div_up(256ull * s.width, 32), 256, 0, stream>>>(r);
            launch_check("k_hist_reduce");
        }
        if (profiled) {
            prof.builds += 1;
            if (!dev_left) {  // rows known on the host: rows x (the used features' bin bytes + 4 B gradients + 4 B
                // row id) + the output, 2 x 4 B a bin of the used features
                prof.rows += count;
                prof.bins += static_cast<double>(count) * static_cast<double>(use.columns);
                prof.hist_bytes += static_cast<double>(count) * (static_cast<double>(use.bin_bytes) + 8.0) +
                                   8.0 * static_cast<double>(use.bins);
            }
        }
    }

    HistUse used_columns() const {
        return hist_use([&](uint32_t f) { return used[f] != 0; });
    }

    void check_range(srocm_leaf_range leaf) const {
        uint64_t end = static_cast<uint64_t>(leaf.begin) + leaf.count;
        if (end > part_len)
            fail(SROCM_ERR_DEVICE, "leaf rows " + std::to_string(leaf.begin) + ".." + std::to_string(end) +
                                       " outside the partition of " + std::to_string(part_len) + " rows");
    }

    DevBuf<int64_t> tmp_hist;

    void histogram_to_host(double *out) {
        hip_check(hipMemcpyAsync(h_hist.p, tmp_hist.p, 2 * total_bins * sizeof(int64_t), hipMemcpyDeviceToHost, stream), "read histogram");
    }

    void histogram(srocm_leaf_range leaf, int quantized, double *out, size_t len) {
        require_loaded();
        check_range(leaf);
        ensure_order();
        if (!quantized) fail(SROCM_ERR_UNSUPPORTED, "float-mode histograms run on the cpu backend only");
        if (len != 2 * total_bins) fail(SROCM_ERR_DEVICE, "histogram buffer of " + std::to_string(len) + " values, expected " + std::to_string(2 * total_bins));
        if (!quantized_once) fail(SROCM_ERR_DEVICE, "histogram before quantize");
        tmp_hist.alloc(2 * total_bins);
        h_hist.alloc(2 * total_bins);
        if (leaf.count == 0) {
            std::fill(out, out + len, 0.0);
            return;
        }
        launch_hist(leaf.begin, leaf.count, nullptr, 0, tmp_hist.p, nullptr, used_columns());
        histogram_to_host(out);
        sync();
        for (size_t i = 0; i < len; ++i) out[i] = static_cast<double>(h_hist.p[i]);
    }

    // histogram() into a caller-owned device buffer (i64 {g, h} per bin), with the partials in the scratch array:
    // allocates nothing. The workgroups are capped so their partials fit the scratch, which leaves more rows per
    // workgroup; their i32 sums must still hold max_q * rows (the sizes beyond that are refused).
    void histogram_noalloc(srocm_leaf_range leaf, int64_t *d_out, size_t len, int wait) {
        require_loaded();
        check_range(leaf);
        ensure_order();  // after a boosting call: its buffers are preallocated, so this allocates nothing either
        if (len != 2 * total_bins) fail(SROCM_ERR_DEVICE, "histogram buffer of " + std::to_string(len) + " values, expected " + std::to_string(2 * total_bins));
        if (!d_out) fail(SROCM_ERR_DEVICE, "null histogram buffer");
        if (!quantized_once) fail(SROCM_ERR_DEVICE, "histogram before quantize");
        if (!scratch_at) fail(SROCM_ERR_DEVICE, "no scratch address for this device");
        const uint32_t cap = static_cast<uint32_t>(NOALLOC_SCRATCH_PAIRS / (256ull * max_width));
        const uint32_t grid = std::max<uint32_t>(1, std::min(hist_groups(leaf.count), cap));
        const uint64_t per = div_up(std::max<uint64_t>(div_up(std::max<uint64_t>(leaf.count, 1), grid), HIST_MIN_ROWS), 64) * 64;
        if (static_cast<uint64_t>(std::max(max_gq, max_hq)) * per > 2147483647ull)
            fail(SROCM_ERR_UNSUPPORTED, "a leaf of " + std::to_string(leaf.count) + " rows over at most " + std::to_string(cap) +
                                            " workgroups (the scratch's limit) could overflow their 32-bit sums at " +
                                            std::to_string(std::max(max_gq, max_hq)) + " quantized units");
        if (leaf.count == 0) {
            k_zero_i64<<<grid_rows(len), 256, 0, stream>>>(d_out, len);
            launch_check("k_zero_i64");
        } else {
            launch_hist_into(leaf.begin, leaf.count, nullptr, 0, d_out, nullptr, used_columns(),
                             reinterpret_cast<int32_t *>(scratch_at), grid, false);
        }
        if (wait) sync();
    }


    // ------------------------------------------------------------------------------------------------
    // partition
    // ------------------------------------------------------------------------------------------------

    PartArgs part_args(uint32_t begin, uint32_t count) {
        PartArgs a{};
        a.src = part.p;
        a.dst = part2.p;
        a.block_left = block_left.p;
        a.dev_left = scalars.p;
        a.begin = begin;
        a.count = count;
        return a;
    }

    // `count` is the rows to partition.
    void run_partition(const PartArgs &a, uint32_t count) {
        uint32_t grid = std::max<uint32_t>(1, std::min<uint32_t>(cus, div_up(count, 1024)));
        hipEvent_t e0 = nullptr, e1 = nullptr;
        if (prof.on) {
            e0 = event();
            e1 = event();
            hip_check(hipEventRecord(e0, stream), "event");
        }
        k_part_count<<<grid, 256, 0, stream>>>(a);
        launch_check("k_part_count");
        k_part_scatter<<<grid, 256, 0, stream>>>(a);
        launch_check("k_part_scatter");
        // the trait's partition is in place: bring the range back into the first buffer
        k_copy_u32<<<std::max<uint32_t>(1, std::min<uint32_t>(div_up(count, 256), cus * 8)), 256, 0, stream>>>(part2.p, part.p, a.begin,
                                                                                                        count);
        launch_check("k_copy_u32");
        if (prof.on) {
            hip_check(hipEventRecord(e1, stream), "event");
            prof.part_events.emplace_back(e0, e1);
            prof.part_launches += 1;
            prof.part_rows += count;
        }
    }

    // Enqueues the stable partition of `leaf` by `split`; the left count lands in scalars[0].
    void enqueue_partition(srocm_leaf_range leaf, const srocm_bin_split &split) {
        if (split.group >= group_col_nt.size()) fail(SROCM_ERR_DEVICE, "split on missing group " + std::to_string(split.group));
        if (split.column >= group_col_nt[split.group].size() || group_col_nt[split.group][split.column] < 0)
            fail(SROCM_ERR_DEVICE, "split on a column without a feature");
        int32_t nt = group_col_nt[split.group][split.column];
        if (leaf.count == 0) {
            hip_check(hipMemsetAsync(scalars.p, 0, 4, stream), "zero left");
            return;
        }
        PartArgs a = part_args(leaf.begin, leaf.count);
        a.col = train.col.p + static_cast<size_t>(nt) * rows * (col16 ? 2 : 1);
        a.col16 = col16;
        a.wide = group_bits[split.group] == 16 ? 1u : 0u;
        std::memcpy(a.left_bins, split.left_bins, sizeof(a.left_bins));
        run_partition(a, leaf.count);
    }

    uint32_t partition(srocm_leaf_range leaf, const srocm_bin_split &split) {
        require_loaded();
        check_range(leaf);
        ensure_order();
        enqueue_partition(leaf, split);
        hip_check(hipMemcpyAsync(h_u32.p, scalars.p, 4, hipMemcpyDeviceToHost, stream), "read left count");
        sync();
        return h_u32.p[0];
    }

    uint32_t partition_and_histogram(srocm_leaf_range leaf, const srocm_bin_split &split, uint32_t side, int quantized,
                                     double *out, size_t len) {
        require_loaded();
        check_range(leaf);
        ensure_order();
        if (!quantized) fail(SROCM_ERR_UNSUPPORTED, "float-mode histograms run on the cpu backend only");
        if (len != 2 * total_bins) fail(SROCM_ERR_DEVICE, "histogram buffer of " + std::to_string(len) + " values, expected " + std::to_string(2 * total_bins));
        if (side > 1) fail(SROCM_ERR_DEVICE, "bad side");
        tmp_hist.alloc(2 * total_bins);
        h_hist.alloc(2 * total_bins);
        enqueue_partition(leaf, split);
        if (leaf.count) launch_hist(leaf.begin, leaf.count, scalars.p, side, tmp_hist.p, nullptr, used_columns());
        else hip_check(hipMemsetAsync(tmp_hist.p, 0, 2 * total_bins * 8, stream), "zero histogram");
        histogram_to_host(out);
        hip_check(hipMemcpyAsync(h_u32.p, scalars.p, 4, hipMemcpyDeviceToHost, stream), "read left count");
        sync();
        for (size_t i = 0; i < len; ++i) out[i] = static_cast<double>(h_hist.p[i]);
        return h_u32.p[0];
    }

    // ------------------------------------------------------------------------------------------------
    // leaf sums, add_tree, scores
    // ------------------------------------------------------------------------------------------------

    void leaf_sums(const srocm_leaf_range *leaves, uint32_t n, float gs, float hs, int64_t *out) {
        require_loaded();
        for (uint32_t i = 0; i < n; ++i) check_range(leaves[i]);
        ensure_order();
        if (n == 0) return;
        std::vector<LeafJob> jobs(n);
        uint32_t maxc = 0;
        for (uint32_t i = 0; i < n; ++i) {
            jobs[i] = LeafJob{leaves[i].begin, leaves[i].count, i};
            maxc = std::max(maxc, leaves[i].count);
        }
        d_leaf_jobs.alloc(n);
        d_leaf_out.alloc(2 * n);
        hip_check(hipMemcpyAsync(d_leaf_jobs.p, jobs.data(), n * sizeof(LeafJob), hipMemcpyHostToDevice, stream), "upload leaves");
        hip_check(hipMemsetAsync(d_leaf_out.p, 0, 2 * n * 8, stream), "zero sums");
        uint32_t chunk = 8192;
        dim3 grid(std::max<uint32_t>(1, div_up(maxc, chunk)), n);
        k_leaf_sums<<<grid, 256, 0, stream>>>(grad.p, hess.p, part.p, d_leaf_jobs.p, gs, hs, d_leaf_out.p, chunk);
        launch_check("k_leaf_sums");
        Pinned<unsigned long long> &h = h_sums;
        h.alloc(2 * n);
        hip_check(hipMemcpyAsync(h.p, d_leaf_out.p, 2 * n * 8, hipMemcpyDeviceToHost, stream), "read sums");
        sync();
        for (uint32_t i = 0; i < 2 * n; ++i) out[i] = static_cast<int64_t>(h.p[i]);
    }

    // A tree's nodes, checked, into d_nodes (through pinned staging, rewritten only after a sync).
    void upload_nodes(const srocm_device_node *nodes, uint32_t nn, uint32_t nl) {
        if (nl == 0 || nl != nn + 1) fail(SROCM_ERR_DEVICE, "tree with " + std::to_string(nn) + " nodes and " + std::to_string(nl) + " leaves");
        h_nodes.alloc(std::max<uint32_t>(nn, 1));
        DevNode *dn = h_nodes.p;
        for (uint32_t k = 0; k < nn; ++k) {
            const srocm_device_node &n = nodes[k];
            if (n.split.group >= group_col_nt.size() || n.split.column >= group_col_nt[n.split.group].size() ||
                group_col_nt[n.split.group][n.split.column] < 0)
                fail(SROCM_ERR_DEVICE, "malformed device tree");
            for (int32_t c : {n.left, n.right}) {
                bool bad = c >= 0 ? (static_cast<uint32_t>(c) <= k || static_cast<uint32_t>(c) >= nn) : (static_cast<uint32_t>(~c) >= nl);
                if (bad) fail(SROCM_ERR_DEVICE, "malformed device tree");
            }
            std::memcpy(dn[k].left_bins, n.split.left_bins, sizeof(dn[k].left_bins));
            dn[k].feature = static_cast<uint32_t>(group_col_nt[n.split.group][n.split.column]);
            dn[k].left = n.left;
            dn[k].right = n.right;
            dn[k].wide = group_bits[n.split.group] == 16 ? 1u : 0u;
        }
        d_nodes.alloc(std::max<uint32_t>(nn, 1));
        if (nn) hip_check(hipMemcpyAsync(d_nodes.p, dn, nn * sizeof(DevNode), hipMemcpyHostToDevice, stream), "upload tree");
    }

    void upload_leaf_values(const float *lv, uint32_t nl) {
        h_lv.alloc(nl);
        std::copy(lv, lv + nl, h_lv.p);
        d_leaf_values.alloc(nl);
        hip_check(hipMemcpyAsync(d_leaf_values.p, h_lv.p, nl * sizeof(float), hipMemcpyHostToDevice, stream), "upload leaves");
    }

    // scores += the uploaded tree's leaf values, through a walk per row, or (train, leaf_of) the leaves k_tree_leaves
    // recorded
    void apply_tree(DevData &d, uint32_t nn, float v0, bool from_leaf_of) {
        if (d.rows == 0) return;
        if (nn == 0) k_add_const<<<grid_rows(d.rows), 256, 0, stream>>>(d.scores.p, d.rows, v0);
        else if (from_leaf_of) k_add_leaf_values<<<grid_rows(d.rows), 256, 0, stream>>>(leaf_of.p, d_leaf_values.p, d.scores.p, d.rows, nullptr);
        else k_add_tree<<<grid_rows(d.rows), 256, 0, stream>>>(d.col.p, col16, d.rows, d_nodes.p, d_leaf_values.p, d.scores.p, nullptr);
        launch_check("k_add_tree");
    }

    void add_tree(const srocm_device_node *nodes, uint32_t nn, const float *lv, uint32_t nl) {
        require_loaded();
        upload_nodes(nodes, nn, nl);
        upload_leaf_values(lv, nl);
        apply_tree(train, nn, lv[0], false);
        for (auto &v : valid) apply_tree(v, nn, lv[0], false);
        sync();  // the staging is rewritten by the next call
    }

    // k_tree_leaves<MAXL, COL16> on as many blocks as the compute units hold at once (the runtime's occupancy for the
    // kernel), or fewer when the rows take fewer
    template <uint32_t MAXL, bool COL16>
    void launch_tree_leaves(const TreeLeavesArgs &a) {
        constexpr uint32_t threads = tl_threads<MAXL>();
        static const int per_cu = [] {
            int n = 0;
            hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_tree_leaves<MAXL, COL16>, threads, 0), "occupancy");
            return n > 0 ? n : 1;
        }();
        const uint32_t grid = static_cast<uint32_t>(std::min<uint64_t>(static_cast<uint64_t>(per_cu) * cus,
                                                                        div_up(rows, static_cast<uint64_t>(tl_rows<MAXL>()) * threads)));
        k_tree_leaves<MAXL, COL16><<<grid, threads, 0, stream>>>(a);
    }

    // k_tree_leaves for trees of up to max_leaves leaves (the gate, when set, holds the actual count)
    void launch_tree_leaves(const TreeLeavesArgs &a, uint32_t max_leaves) {
        if (max_leaves <= LEAVES_SMALL) {
            if (a.col16) launch_tree_leaves<LEAVES_SMALL, true>(a);
            else launch_tree_leaves<LEAVES_SMALL, false>(a);
        } else if (max_leaves <= GROW_MAX_LEAVES) {
            if (a.col16) launch_tree_leaves<GROW_MAX_LEAVES, true>(a);
            else launch_tree_leaves<GROW_MAX_LEAVES, false>(a);
        } else {
            fail(SROCM_ERR_UNSUPPORTED, "a tree of " + std::to_string(max_leaves) + " leaves; the row walk takes up to " +
                                            std::to_string(GROW_MAX_LEAVES));
        }
        launch_check("k_tree_leaves");
    }

    // The uploaded tree's leaf of every training row (leaf_of) and, when `sums` is set, the leaves' fixed-point
    // gradient sums over the in-bag rows, as leaf_sums over the grown tree's leaves gives them.
    void tree_leaves(uint32_t nn, uint32_t nl, const srocm_bag &bag, float gs, float hs, int64_t *sums) {
        leaf_of.alloc(rows);
        TreeLeavesArgs a{};
        a.colbins = train.col.p;
        a.col16 = col16;
        a.rows = rows;
        a.nodes = d_nodes.p;
        a.nn = nn;
        a.nl = nl;
        a.leaf_of = leaf_of.p;
        if (sums) {
            d_leaf_out.alloc(2 * nl);
            hip_check(hipMemsetAsync(d_leaf_out.p, 0, 2 * nl * 8, stream), "zero sums");
            a.grad = grad.p;
            a.hess = hess.p;
            a.gs = gs;
            a.hs = hs;
            a.sums = reinterpret_cast<unsigned long long *>(d_leaf_out.p);
            a.bag = bag.kind == SROCM_BAG_BERNOULLI ? 1u : 0u;
            a.bag_seed = bag.seed;
            a.bag_round = bag.round;
            a.row_offset = row_offset;
            a.fraction = bag.fraction;
        }
        launch_tree_leaves(a, nl);
        if (!sums) return;
        Pinned<unsigned long long> &h = h_sums;
        h.alloc(2 * nl);
        hip_check(hipMemcpyAsync(h.p, d_leaf_out.p, 2 * nl * 8, hipMemcpyDeviceToHost, stream), "read sums");
        sync();
        for (uint32_t i = 0; i < 2 * nl; ++i) sums[i] = static_cast<int64_t>(h.p[i]);
    }

    DevData &dataset(uint32_t i) {
        if (i == 0) return train;
        if (i - 1 >= valid.size()) fail(SROCM_ERR_DEVICE, "no dataset " + std::to_string(i));
        return valid[i - 1];
    }

    void init_scores(uint32_t i, double value) {
        require_loaded();
        DevData &d = dataset(i);
        if (d.rows) {
            k_fill_f32<<<grid_rows(d.rows), 256, 0, stream>>>(d.scores.p, d.rows, static_cast<float>(value));
            launch_check("k_fill_f32");
        }
    }

    void scores(uint32_t i, float *out, size_t len) {
        require_loaded();
        DevData &d = dataset(i);
        if (len != d.rows) fail(SROCM_ERR_DEVICE, "scores buffer of " + std::to_string(len) + " values, expected " + std::to_string(d.rows));
        if (len) hip_check(hipMemcpyAsync(out, d.scores.p, len * 4, hipMemcpyDeviceToHost, stream), "read scores");
        sync();
    }

    // ------------------------------------------------------------------------------------------------
    // device split search (split.rs:919-961)
    // ------------------------------------------------------------------------------------------------

    static SplitCfgDev cfg_dev(const srocm_split_config &c) {
        return SplitCfgDev{c.min_data_in_leaf, c.min_sum_hessian_in_leaf, c.lambda_l1, c.lambda_l2, c.min_gain_to_split,
                           c.max_cat_to_onehot, c.max_cat_threshold, c.cat_l2, c.cat_smooth, c.min_data_per_group};
    }

    // ------------------------------------------------------------------------------------------------
    // histogram slots: the learner's histograms kept on the device (learner.rs:121-352 over the trait calls, with
    // the subtraction of learner.rs:356-371 and the split search reading them where they are)
    DevBuf<int64_t> hslots;   // num_hslots histograms of 2 * total_bins int64 units
    uint32_t num_hslots = 0;

    int64_t *slot_ptr(uint32_t slot) {
        if (slot >= num_hslots)
            fail(SROCM_ERR_DEVICE, "histogram slot " + std::to_string(slot) + " of " + std::to_string(num_hslots));
        return hslots.p + static_cast<size_t>(slot) * 2 * total_bins;
    }

    void hist_slots(uint32_t n) {
        require_loaded();
        hslots.alloc(static_cast<size_t>(std::max<uint32_t>(n, 1)) * 2 * total_bins);
        num_hslots = n;
    }

    void histogram_slot(srocm_leaf_range leaf, uint32_t slot) {
        require_loaded();
        check_range(leaf);
        ensure_order();
        if (!quantized_once) fail(SROCM_ERR_DEVICE, "histogram before quantize");
        int64_t *d = slot_ptr(slot);
        if (leaf.count) launch_hist(leaf.begin, leaf.count, nullptr, 0, d, nullptr, used_columns());
        else hip_check(hipMemsetAsync(d, 0, 2 * total_bins * 8, stream), "zero histogram");
    }

    uint32_t partition_and_histogram_slot(srocm_leaf_range leaf, const srocm_bin_split &split, uint32_t side, uint32_t slot) {
        require_loaded();
        check_range(leaf);
        ensure_order();
        if (side > 1) fail(SROCM_ERR_DEVICE, "bad side");
        if (!quantized_once) fail(SROCM_ERR_DEVICE, "histogram before quantize");
        int64_t *d = slot_ptr(slot);
        enqueue_partition(leaf, split);
        if (leaf.count) launch_hist(leaf.begin, leaf.count, scalars.p, side, d, nullptr, used_columns());
        else hip_check(hipMemsetAsync(d, 0, 2 * total_bins * 8, stream), "zero histogram");
        hip_check(hipMemcpyAsync(h_u32.p, scalars.p, 4, hipMemcpyDeviceToHost, stream), "read left count");
        sync();
        return h_u32.p[0];
    }

    // learner.rs:365-367: the parent's slot becomes parent - built, the other child's histogram (exact integers)
    void subtract(uint32_t parent, uint32_t child) {
        require_loaded();
        if (parent == child) fail(SROCM_ERR_DEVICE, "a slot subtracted from itself");
        int64_t *p = slot_ptr(parent);
        const int64_t *c = slot_ptr(child);
        k_sub_i64<<<grid_rows(2 * total_bins), 256, 0, stream>>>(p, c, 2 * total_bins);
        launch_check("k_sub_i64");
    }

    void read_slot(uint32_t slot, double *out, size_t len) {
        require_loaded();
        if (len != 2 * total_bins) fail(SROCM_ERR_DEVICE, "histogram buffer of " + std::to_string(len) + " values, expected " + std::to_string(2 * total_bins));
        const int64_t *d = slot_ptr(slot);
        h_hist.alloc(2 * total_bins);
        hip_check(hipMemcpyAsync(h_hist.p, d, 2 * total_bins * 8, hipMemcpyDeviceToHost, stream), "read histogram slot");
        sync();
        for (size_t i = 0; i < len; ++i) out[i] = static_cast<double>(h_hist.p[i]);
    }

    void find_best_split_slot(uint32_t slot, const srocm_feature *features, uint32_t num_features, const uint8_t *evaluate,
                              const srocm_sums &sums, double sg, double sh, const srocm_split_config &cfg,
                              srocm_split_info *out, uint8_t *splittable) {
        require_loaded();
        find_best_split_dev(slot_ptr(slot), 2 * total_bins, features, num_features, evaluate, sums, sg, sh, cfg, out, splittable);
    }

    // split.rs:919-961 on a host histogram over an explicit feature table (no loaded dataset needed)
    void find_best_split(const double *hist, size_t len, const srocm_feature *features, uint32_t num_features,
                         const uint8_t *evaluate, const srocm_sums &sums, double sg, double sh,
                         const srocm_split_config &cfg, srocm_split_info *out, uint8_t *splittable) {
        std::vector<int64_t> units(len);
        for (size_t i = 0; i < len; ++i) units[i] = static_cast<int64_t>(hist[i]);
        DevBuf<int64_t> dh;
        dh.alloc(std::max<size_t>(len, 1));
        if (len) hip_check(hipMemcpyAsync(dh.p, units.data(), len * 8, hipMemcpyHostToDevice, stream), "upload histogram");
        find_best_split_dev(dh.p, len, features, num_features, evaluate, sums, sg, sh, cfg, out, splittable);
    }

    // find_best_split over `len` int64 units on the device (an uploaded host histogram, or a histogram slot)
    void find_best_split_dev(const int64_t *dh, size_t len, const srocm_feature *features, uint32_t num_features,
                             const uint8_t *evaluate, const srocm_sums &sums, double sg, double sh,
                             const srocm_split_config &cfg, srocm_split_info *out, uint8_t *splittable) {
        std::vector<FeatDev> fd(num_features);
        for (uint32_t f = 0; f < num_features; ++f) {
            const srocm_feature &m = features[f];
            if (m.num_bins > 1024 || (m.num_bins > 256 && m.kind != SROCM_BINS_NUMERICAL))
                fail(SROCM_ERR_UNSUPPORTED, "a feature of more than 1024 bins, or a categorical one of more than 256");
            if (m.num_bins && static_cast<uint64_t>(m.hist_offset) + m.num_bins > len / 2)
                fail(SROCM_ERR_DEVICE, "feature " + std::to_string(f) + " lies outside the histogram");
            fd[f] = FeatDev{m.num_bins, m.hist_offset, m.kind, m.nan_bin, 0u, m.num_bins > 256 ? 1u : 0u};
        }
        DevBuf<FeatDev> dfd;
        DevBuf<ScanJob> dj;
        DevBuf<FeatCand> dc;
        DevBuf<SplitOut> dso;
        DevBuf<uint8_t> dsp, dev, dorder;
        dorder.alloc(static_cast<size_t>(std::max<uint32_t>(num_features, 1)) * 256);
        dfd.alloc(std::max<uint32_t>(num_features, 1));
        dj.alloc(1);
        dc.alloc(std::max<uint32_t>(num_features, 1));
        dso.alloc(1);
        dsp.alloc(std::max<uint32_t>(num_features, 1));
        dev.alloc(std::max<uint32_t>(num_features, 1));
        if (num_features) {
            hip_check(hipMemcpyAsync(dfd.p, fd.data(), num_features * sizeof(FeatDev), hipMemcpyHostToDevice, stream), "upload features");
            hip_check(hipMemcpyAsync(dev.p, evaluate, num_features, hipMemcpyHostToDevice, stream), "upload evaluate");
        }
        ScanJob job{dh, sums.grad, sums.hess, sums.count, dc.p};
        hip_check(hipMemcpyAsync(dj.p, &job, sizeof(job), hipMemcpyHostToDevice, stream), "upload job");
        if (num_features) {
            // numerical byte features of 2..64 bins go in scan units of several (k_split_scan_seg), as in a tree
            std::vector<uint8_t> seg(num_features, 0);
            std::vector<int32_t> ufeat;
            std::vector<uint32_t> usegl;
            for (uint32_t segl : {4u, 16u}) {
                std::vector<int32_t> members;
                for (uint32_t f = 0; f < num_features; ++f) {
                    const FeatDev &x = fd[f];
                    if (x.kind == SROCM_BINS_NUMERICAL && !x.wide && x.num_bins >= 2 && x.num_bins <= 64 &&
                        (x.num_bins > 16 ? 16u : 4u) == segl) {
                        members.push_back(static_cast<int32_t>(f));
                        seg[f] = 1;
                    }
                }
                const size_t per = 64 / segl;
                for (size_t b = 0; b < members.size(); b += per) {
                    for (size_t k = 0; k < UNIT_FEATS; ++k) ufeat.push_back(k < per && b + k < members.size() ? members[b + k] : -1);
                    usegl.push_back(segl);
                }
            }
            DevBuf<uint8_t> dseg;
            DevBuf<int32_t> dufeat;
            DevBuf<uint32_t> dusegl;
            dseg.alloc(num_features);
            hip_check(hipMemcpyAsync(dseg.p, seg.data(), num_features, hipMemcpyHostToDevice, stream), "upload scan units");
            dim3 grid(div_up(num_features, 4), 1);
            bool narrow = false, wide = false;
            for (const FeatDev &x : fd) (x.wide ? wide : narrow) = true;
            if (narrow) k_split_scan<false><<<grid, 256, 0, stream>>>(dj.p, dfd.p, dev.p, num_features, cfg_dev(cfg), sg, sh, dorder.p, nullptr, dseg.p);
            if (wide) k_split_scan<true><<<grid, 256, 0, stream>>>(dj.p, dfd.p, dev.p, num_features, cfg_dev(cfg), sg, sh, dorder.p, nullptr);
            launch_check("k_split_scan");
            if (!usegl.empty()) {
                dufeat.alloc(ufeat.size());
                dusegl.alloc(usegl.size());
                hip_check(hipMemcpyAsync(dufeat.p, ufeat.data(), ufeat.size() * 4, hipMemcpyHostToDevice, stream), "upload scan units");
                hip_check(hipMemcpyAsync(dusegl.p, usegl.data(), usegl.size() * 4, hipMemcpyHostToDevice, stream), "upload scan units");
                k_split_scan_seg<<<dim3(div_up(usegl.size(), 4), 1), 256, 0, stream>>>(dj.p, dfd.p, dev.p, dufeat.p, dusegl.p,
                                                                                      static_cast<uint32_t>(usegl.size()), cfg_dev(cfg), sg, sh);
                launch_check("k_split_scan_seg");
            }
            sync();  // the unit buffers are locals
        }
        k_split_select<<<1, 256, 0, stream>>>(dj.p, num_features, cfg_dev(cfg), sg, sh, dso.p, dsp.p);
        launch_check("k_split_select");
        SplitOut o;
        hip_check(hipMemcpyAsync(&o, dso.p, sizeof(o), hipMemcpyDeviceToHost, stream), "read split");
        if (num_features) hip_check(hipMemcpyAsync(splittable, dsp.p, num_features, hipMemcpyDeviceToHost, stream), "read splittable");
        sync();
        to_info(o, out);
        if (o.found && o.rule == RULE_SORTED) {  // the rule's bins in order (split.rs:114-116)
            uint8_t order[256];
            hip_check(hipMemcpy(order, dorder.p + static_cast<size_t>(o.feature) * 256, 256, hipMemcpyDeviceToHost), "read categories");
            for (uint32_t i = 0; i < o.cat_count && i < 256; ++i) out->cat_bins[i] = order[i];
        }
    }

    static void to_info(const SplitOut &o, srocm_split_info *out) {
        std::memset(out, 0, sizeof(*out));
        out->found = o.found;
        if (!o.found) return;
        out->feature = o.feature;
        out->gain = o.gain;
        out->threshold = o.threshold;
        out->default_left = o.default_left;
        out->left = srocm_sums{o.left_grad, o.left_hess, o.left_count};
        out->right = srocm_sums{o.right_grad, o.right_hess, o.right_count};
        out->left_output = o.left_output;
        out->right_output = o.right_output;
        if (o.rule != RULE_NUMERICAL) {
            out->categorical = 1;
            out->num_cat_bins = o.cat_count;
            uint32_t k = 0;  // one-hot: the single bin of the mask
            for (uint32_t b = 0; b < 256 && k < o.cat_count; ++b)
                if ((o.cat_mask[b >> 5] >> (b & 31)) & 1u) out->cat_bins[k++] = b;
        }
    }

    // ------------------------------------------------------------------------------------------------
    // Learner::grow on the device (learner.rs:121-352)
    // ------------------------------------------------------------------------------------------------

    DevBuf<int64_t> pool;             // histogram slots, 2 * total_bins i64 each
    DevBuf<StepPlan> d_plans;         // [2], by step parity
    DevBuf<TLeaf> d_tl;               // the speculative tree's leaves
    DevBuf<TKey> d_tk;
    DevBuf<uint8_t> d_leaf_left;
    DevBuf<uint8_t> d_splittable, d_eval, d_mask;
    std::vector<uint8_t> d_mask_host;  // what d_mask holds (empty: unknown), so an unchanged mask is not uploaded again
    DevBuf<ScanJob> d_jobs;
    DevBuf<FeatCand> d_cands;
    DevBuf<RowRun> d_runs;            // end of a tree: runs of rows to bring into ascending order
    DevBuf<MergeJob> d_merges;        // end of a tree: leaves whose expansion was dropped
    DevBuf<uint32_t> d_starts;
    Pinned<uint8_t> h_fix;            // staging of the runs and merges (rewritten only after a sync)
    // split steps (k_step_rows, k_step_reduce, k_step_scan, k_step_cat, k_step_select)
    DevBuf<int32_t> step_partial;            // per slab: [cus + JMAX][256 * W] {g, h}
    DevBuf<unsigned long long> tile_status;  // per partition tile
    DevBuf<uint32_t> fin_counts;             // the jobs-selected counter of k_step_select
    uint64_t epochs_used = 0;
    uint32_t last_steps = 0;                 // split steps of the last tree (the first guess for the next)
    // The control block, the tree arrays, the leaves' row ranges and the committed leaves' speculative leaves, in one
    // allocation so that the check for the end of a tree brings the tree back with it: 8-byte arrays, then 4-byte
    // arrays, the left-bin masks and the default-left flags, each padded to 8 B.
    struct TreeLayout {
        size_t ctl, iv, iw, lv, lw, ic, lc, leaf_t, sf, lch, rch, lp, ld, tb, sg, lr, lb, dl, bytes;
        explicit TreeLayout(uint32_t L = 0) {
            size_t at = 0;
            auto take = [&](size_t n) { size_t o = at; at += (n + 7) & ~static_cast<size_t>(7); return o; };
            ctl = take(sizeof(GrowCtl));
            iv = take(8ull * L); iw = take(8ull * L); lv = take(8ull * L); lw = take(8ull * L); ic = take(8ull * L); lc = take(8ull * L);
            leaf_t = take(4ull * L); sf = take(4ull * L); lch = take(4ull * L); rch = take(4ull * L); lp = take(4ull * L);
            ld = take(4ull * L); tb = take(4ull * L); sg = take(4ull * L); lr = take(8ull * L); lb = take(32ull * L); dl = take(L);
            bytes = at;
        }
    };
    DevBuf<uint8_t> dtree;
    TreeLayout tree_layout;
    uint32_t grow_capacity = 0;

    uint32_t k1_groups() const { return step_target + JMAX; }  // k_step_rows' grid
    uint32_t scan_blocks() const { return 8 * cus; }   // k_step_scan's grid: four waves a block, a wave per item
    uint32_t reduce_blocks() const { return 8 * cus; } // k_step_reduce's grid

    void ensure_grow(uint32_t L) {
        if (grow_capacity >= L && pool.p) return;
        const uint32_t tcap = grow_tcap(L), nslots = tcap / 2 + 1;
        pool.alloc(static_cast<size_t>(nslots) * 2 * total_bins);
        d_plans.alloc(2);
        d_tl.alloc(tcap);
        d_tk.alloc(tcap);
        d_leaf_left.alloc(L);
        d_splittable.alloc(static_cast<size_t>(tcap) * nf);
        d_eval.alloc(nf);
        d_mask.alloc(nf);
        d_mask_host.clear();
        d_jobs.alloc(1);
        d_cands.alloc(static_cast<size_t>(JMAX) * 2 * nf);
        tree_layout = TreeLayout(L);
        dtree.alloc(tree_layout.bytes);
        // host staging at its largest, so that no tree allocates pinned memory
        h_result.alloc(((static_cast<size_t>(grow_tcap(L)) * sizeof(TLeaf) + 7) & ~static_cast<size_t>(7)) + tree_layout.bytes);
        h_fix.alloc(static_cast<size_t>(grow_tcap(L)) * (sizeof(RowRun) + sizeof(MergeJob) + 8) + 64);
        d_runs.alloc(grow_tcap(L));  // the row-order restore's device lists at their largest too
        d_merges.alloc(L);
        d_starts.alloc(static_cast<size_t>(grow_tcap(L)) + L);
        h_nodes.alloc(L);
        h_lv.alloc(L);
        h_sums.alloc(2 * static_cast<size_t>(L));
        step_partial.alloc(2 * step_partial_pairs);
        tile_status.alloc(div_up(rows, STEP_TILE) + JMAX + 1);
        fin_counts.alloc(1);
        reset_step_state();
        grow_capacity = L;
    }

    // Tile status words carry the step's epoch; the counters are returned to zero by the kernels themselves.
    void reset_step_state() {
        hip_check(hipMemsetAsync(dtree.p + tree_layout.ctl, 0, sizeof(GrowCtl), stream), "zero grow control");
        hip_check(hipMemsetAsync(tile_status.p, 0, tile_status.n * sizeof(unsigned long long), stream), "zero tile status");
        hip_check(hipMemsetAsync(fin_counts.p, 0, fin_counts.n * sizeof(uint32_t), stream), "zero step counters");
        epochs_used = 0;
    }

    GrowState grow_state(const srocm_grow_spec &spec) {
        GrowState g{};
        g.plans = d_plans.p;
        g.tl = d_tl.p;
        g.tk = d_tk.p;
        const TreeLayout &tl = tree_layout;
        uint8_t *tp = dtree.p;
        g.ctl = reinterpret_cast<GrowCtl *>(tp + tl.ctl);
        g.leaf_t = reinterpret_cast<int32_t *>(tp + tl.leaf_t);
        g.leaf_left = d_leaf_left.p;
        g.splittable = d_splittable.p;
        g.jobs = d_jobs.p;
        g.cands = d_cands.p;
        g.evaluate = d_eval.p;
        g.mask = d_mask.p;
        g.feats = dfeats.p;
        g.tree = TreeDev{reinterpret_cast<int32_t *>(tp + tl.sf), reinterpret_cast<uint32_t *>(tp + tl.tb), tp + tl.dl,
                         reinterpret_cast<int32_t *>(tp + tl.lch), reinterpret_cast<int32_t *>(tp + tl.rch),
                         reinterpret_cast<float *>(tp + tl.sg), reinterpret_cast<double *>(tp + tl.iv),
                         reinterpret_cast<double *>(tp + tl.iw), reinterpret_cast<int64_t *>(tp + tl.ic),
                         reinterpret_cast<double *>(tp + tl.lv), reinterpret_cast<double *>(tp + tl.lw),
                         reinterpret_cast<int64_t *>(tp + tl.lc), reinterpret_cast<int32_t *>(tp + tl.lp),
                         reinterpret_cast<int32_t *>(tp + tl.ld), reinterpret_cast<uint32_t *>(tp + tl.lb),
                         reinterpret_cast<uint32_t *>(tp + tl.lr)};
        g.pool = pool.p;
        g.slot_stride = 2 * total_bins;
        g.nf = nf;
        g.num_leaves = spec.num_leaves;
        g.tcap = grow_tcap(spec.num_leaves);
        g.nslots = g.tcap / 2 + 1;
        g.max_depth = spec.max_depth;
        g.cfg = cfg_dev(spec.cfg);
        g.sg = spec.grad_scale;
        g.sh = spec.hess_scale;
        g.dsc = grow_dsc;
        g.target_groups = step_target;
        g.jcap = grow_jcap(spec.num_leaves);
        g.ncg = ncg;
        g.nsg = nsg;
        g.flush_rows = flush_rows();
        // a workgroup's i32 sums take at most (2^31 - 1) / max_q rows
        const uint64_t mq = static_cast<uint64_t>(std::max<int64_t>(std::max(max_gq, max_hq), 1));
        g.tile_cap = static_cast<uint32_t>(std::max<uint64_t>(std::min<uint64_t>((2147483647ull / mq) / STEP_TILE, 1u << 30), 1));
        g.hist_weight = STEP_HIST_WEIGHT;
        g.sparse_weight = STEP_SPARSE_WEIGHT;
        return g;
    }

    // `final_order`: leave every leaf's rows ascending in the partition (the reference's order); without it the rows
    // of each leaf are only grouped, which is all the boosting loop needs before the next tree resets them.
    // `after_steps` (when set) is called after each batch of split steps is launched, before the host waits on it.
    void grow(const srocm_grow_spec &spec, HostTree &tree, std::vector<srocm_bin_split> &splits, std::vector<GrowLeaf> &leaves,
              bool final_order = true, const std::function<void(const GrowState &)> *after_steps = nullptr);
    void restore_order(uint32_t n, uint32_t ntent, const int32_t *lt);
    // The boosting loop's last tree leaves its row order to be restored by the first call that reads the partition
    // (ensure_order; a reset of the partition drops it), so a loop run an iteration at a time does not pay for it.
    struct PendingOrder {
        bool on = false;
        uint32_t n = 0, ntent = 0;
        std::vector<int32_t> lt;
    };
    bool defer_order = false;
    PendingOrder pending_order;
    void ensure_order() {
        if (!pending_order.on) return;
        pending_order.on = false;
        restore_order(pending_order.n, pending_order.ntent, pending_order.lt.data());
    }

    void copy_tree(const HostTree &t, const std::vector<GrowLeaf> &leaves, srocm_grown_tree *out) const {
        if (out->capacity_leaves < t.num_leaves) fail(SROCM_ERR_DEVICE, "grown tree has more leaves than the output holds");
        out->num_leaves = t.num_leaves;
        uint32_t ni = t.num_leaves - 1;
        auto cp = [](auto *dst, const auto &v, size_t n) {
            if (dst) std::copy(v.begin(), v.begin() + static_cast<long>(n), dst);
        };
        cp(out->split_feature, t.split_feature, ni);
        cp(out->threshold_bin, t.threshold_bin, ni);
        cp(out->default_left, t.default_left, ni);
        cp(out->left_child, t.left_child, ni);
        cp(out->right_child, t.right_child, ni);
        cp(out->split_gain, t.split_gain, ni);
        cp(out->internal_value, t.internal_value, ni);
        cp(out->internal_weight, t.internal_weight, ni);
        cp(out->internal_count, t.internal_count, ni);
        cp(out->leaf_value, t.leaf_value, t.num_leaves);
        cp(out->leaf_weight, t.leaf_weight, t.num_leaves);
        cp(out->leaf_count, t.leaf_count, t.num_leaves);
        cp(out->leaf_parent, t.leaf_parent, t.num_leaves);
        cp(out->leaf_depth, t.leaf_depth, t.num_leaves);
        cp(out->left_bins, t.left_bins, static_cast<size_t>(ni) * 8);
        if (out->leaf_range)
            for (uint32_t i = 0; i < t.num_leaves && i < leaves.size(); ++i) out->leaf_range[i] = leaves[i].range;
    }

    // ------------------------------------------------------------------------------------------------
    // boosting (boosting.rs:83-324)
    // ------------------------------------------------------------------------------------------------

    double init_score_value = 0.0;
    uint32_t trees_added = 0;

    double boost_init(const srocm_train_params &p);
    uint32_t boost(const srocm_train_params &p, uint32_t first, uint32_t count, srocm_grown_tree *trees);

    // profiling
    void profile(int enable) {
        settle_profile();
        prof.on = enable != 0;
        prof.sectors = enable == 2;
        prof.reset();
        if (prof.sectors) {
            prof.sector_counts.alloc(10);
            hip_check(hipMemsetAsync(prof.sector_counts.p, 0, 10 * sizeof(unsigned long long), stream), "zero sectors");
            const uint64_t words = sector_bit_words();
            prof.sector_bits.alloc(words);
            hip_check(hipMemsetAsync(prof.sector_bits.p, 0, words * 4, stream), "zero sector bits");
        }
    }
    uint64_t sectors_per_col() const { return div_up(std::max<uint64_t>(rows, 1), col16 ? 64 : 128); }
    uint64_t sector_bit_words() const { return div_up(static_cast<uint64_t>(nt_feat.size()) * sectors_per_col(), 32); }
    // after a split step's k_step_rows launches: the distinct sectors its gathers touch (measurement only)
    void sector_model(uint32_t parity) {
        if (!prof.sectors) return;
        k_sector_model<<<dim3(1, JMAX), 256, 0, stream>>>(d_plans.p + parity, part.p, part2.p, col16, prof.sector_bits.p,
                                                         sectors_per_col(), d_fmt.p, prof.sector_counts.p);
        launch_check("k_sector_model");
        k_sector_bits<<<std::min<uint64_t>(div_up(sector_bit_words(), 256), cus * 4), 256, 0, stream>>>(
            prof.sector_bits.p, sector_bit_words(), prof.sector_counts.p);
        launch_check("k_sector_bits");
    }
    void settle_profile() {
        sync();
        if (prof.sectors && prof.sector_counts.p) {
            unsigned long long c[10];
            hip_check(hipMemcpy(c, prof.sector_counts.p, sizeof(c), hipMemcpyDeviceToHost), "read sectors");
            for (int k = 0; k < 10; ++k) prof.sector[k] += static_cast<double>(c[k]);
            hip_check(hipMemset(prof.sector_counts.p, 0, sizeof(c)), "zero sectors");
        }
        auto settle = [&](std::vector<std::pair<hipEvent_t, hipEvent_t>> &events, double &total) {
            for (auto &e : events) {
                float ms = 0;
                hip_check(hipEventElapsedTime(&ms, e.first, e.second), "event elapsed");
                total += ms;
                prof.pool.push_back(e.first);
                prof.pool.push_back(e.second);
            }
            events.clear();
        };
        settle(prof.hist_events, prof.hist_ms);
        settle(prof.step_events, prof.step_ms);
        settle(prof.part_events, prof.part_ms);
    }
};

// One feature's bins from its group's rows (a byte, two little-endian bytes, or half a byte: `column` counts 4-bit
// slots, low half first) into its column-major bins and its slab column.
__global__ void k_repack(const uint8_t *__restrict__ src, uint32_t stride, uint32_t column, uint32_t bits,
                         uint64_t n, RepackTo to) {
    for (uint64_t r = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; r < n; r += (uint64_t)gridDim.x * blockDim.x) {
        const uint8_t *row = src + r * stride;
        uint32_t b;
        if (bits == 16) b = static_cast<uint32_t>(row[column]) | (static_cast<uint32_t>(row[column + 1]) << 8);
        else if (bits == 4) b = (static_cast<uint32_t>(row[column >> 1]) >> (4 * (column & 1u))) & 15u;
        else b = row[column];
        if (to.bad && b >= to.num_bins) *to.bad = 1u;  // every writer stores the same value
        if (!to.col) {
        } else if (to.col16) {
            reinterpret_cast<uint16_t *>(to.col)[r] = static_cast<uint16_t>(b);
        } else {
            to.col[r] = static_cast<uint8_t>(b);
        }
        if (!to.slab) continue;
        uint8_t *dst = to.slab + r * to.row_bytes;
        if (to.slab_wide) reinterpret_cast<uint16_t *>(dst)[to.slab_col] = static_cast<uint16_t>(b);
        else dst[to.slab_col] = static_cast<uint8_t>(b);
    }
}

void Context::repack(const uint8_t *src, uint32_t stride, uint32_t column, uint32_t bits, uint64_t n,
                     const RepackTo &to) {
    k_repack<<<grid_rows(n), 256, 0, stream>>>(src, stride, column, bits, n, to);
    launch_check("k_repack");
}

// objective/regression.rs:70-93 and objective/binary.rs:27-50 on the device; maxima as cpu.rs:774-778.
std::pair<double, double> Context::compute_gradients() {
    launch_gradients(false);
    if (rank_factors_vetoed()) launch_gradients(true);
    return read_maxima();
}

void Context::launch_gradients(bool host_factors) {
    require_loaded();
    rank_flag_pending = false;
    if (!maxima_clear) hip_check(hipMemsetAsync(maxima.p, 0, 8 * MAX_SLOTS, stream), "zero maxima");
    maxima_clear = false;
    if (rows && objective == SROCM_OBJ_LAMBDARANK) {
        ranking_gradients(host_factors);
    } else if (rows) {
        const float *w = has_weight ? weight.p : nullptr;
        if (objective == SROCM_OBJ_REGRESSION)
            k_grad_regression<<<grid_rows(rows), 256, 0, stream>>>(train.scores.p, label.p, w, grad.p, hess.p, rows, maxima.p);
        else
            k_grad_binary<<<grid_rows(rows), 256, 0, stream>>>(train.scores.p, label.p, w, grad.p, hess.p, rows, sigmoid, maxima.p);
        launch_check("k_grad");
    }
}

// learner.rs:121-352 on the device: split steps are enqueued without waiting; the device replays the reference's
// leaf order, expands leaves (speculatively beyond the next one), partitions, histograms the smaller children,
// subtracts, searches the children and writes the tree. The host checks for the end of the tree once per batch of
// steps (sized by the last tree's step count), reads the finished tree, and enqueues the final row order.
void Context::grow(const srocm_grow_spec &spec, HostTree &tree, std::vector<srocm_bin_split> &splits,
                   std::vector<GrowLeaf> &leaves, bool final_order,
                   const std::function<void(const GrowState &)> *after_steps) {
    require_loaded();
    if (!quantized_once) fail(SROCM_ERR_DEVICE, "grow before quantize");
    check_range(spec.root);
    ensure_order();
    if (spec.num_leaves < 1) fail(SROCM_ERR_CONFIG, "num_leaves must be positive");
    if (spec.num_leaves > GROW_MAX_LEAVES)
        fail(SROCM_ERR_UNSUPPORTED, "device growth takes num_leaves up to " + std::to_string(GROW_MAX_LEAVES));
    const uint32_t L = spec.num_leaves;
    std::vector<uint8_t> mask(spec.feature_mask, spec.feature_mask + nf);
    ensure_grow(L);
    int32_t sums_feature = -1;
    for (uint32_t f = 0; f < nf; ++f)
        if (feats[f].num_bins) {
            sums_feature = static_cast<int32_t>(f);
            break;
        }
    const srocm_split_config &cfg = spec.cfg;
    auto depth_allows = [&](int32_t d) { return spec.max_depth <= 0 || d < spec.max_depth; };
    bool root_searched = sums_feature >= 0 && depth_allows(0) && spec.root_count >= 2 * cfg.min_data_in_leaf;
    GrowState g = grow_state(spec);
    g.sums_feature = sums_feature < 0 ? 0u : static_cast<uint32_t>(sums_feature);
    if (epochs_used + L > (1ull << 29)) reset_step_state();  // tile status epochs are 30 bits wide
    epochs_used += L;
    if (mask != d_mask_host) {  // (feature_fraction 1 keeps one mask for every tree)
        h_stage.alloc(nf + 64);
        std::memcpy(h_stage.p, mask.data(), nf);
        hip_check(hipMemcpyAsync(d_mask.p, h_stage.p, nf, hipMemcpyHostToDevice, stream), "upload mask");
        d_mask_host = mask;
    }
    k_grow_init<<<1, 64, 0, stream>>>(g, spec.root.begin, spec.root.count, spec.root_count, root_searched ? 1u : 0u);
    launch_check("k_grow_init");
    // small units travel beside the row ids as one-byte codes (packed_code), so the split steps' histograms read them
    // with the rows instead of gathering the packed words
    const bool codes = !q32 && max_gq <= CODE_MAX_G && max_hq <= CODE_MAX_H && root_searched && spec.root.count;
    if (codes) {
        codes0.alloc(rows);
        codes1.alloc(rows);
        k_gh_codes<<<std::min<uint32_t>(div_up(spec.root.count, 256), cus * 8), 256, 0, stream>>>(
            part.p, packed.p, spec.root.begin, spec.root.count, codes0.p);
        launch_check("k_gh_codes");
    }
    const HistUse used_root = hist_use([&](uint32_t f) { return mask[f] || static_cast<int32_t>(f) == sums_feature; });
    // the tree block comes back with every check for the end of the tree
    const TreeLayout &lay = tree_layout;
    const size_t tl_max = (static_cast<size_t>(grow_tcap(L)) * sizeof(TLeaf) + 7) & ~static_cast<size_t>(7);
    h_result.alloc(tl_max + lay.bytes);
    uint8_t *hb = h_result.p + tl_max;
    auto read_ctl = [&]() {
        hip_check(hipMemcpyAsync(hb, dtree.p, lay.bytes, hipMemcpyDeviceToHost, stream), "read tree");
        sync();
        return *reinterpret_cast<const GrowCtl *>(hb + lay.ctl);
    };
    GrowCtl hc{};
    if (root_searched) {
        // the root histogram goes into slot 0
        launch_hist(spec.root.begin, spec.root.count, nullptr, 0, pool.p, nullptr, used_root);
        k_root_prep<<<1, 256, 0, stream>>>(g);
        launch_check("k_root_prep");
        if (has_narrow)
            k_split_scan<false><<<dim3(div_up(nf, 4), 1), 256, 0, stream>>>(d_jobs.p, dfeats.p, d_eval.p, nf, g.cfg, g.sg, g.sh, nullptr, g.dsc);
        if (has_wide)
            k_split_scan<true><<<dim3(div_up(nf, 4), 1), 256, 0, stream>>>(d_jobs.p, dfeats.p, d_eval.p, nf, g.cfg, g.sg, g.sh, nullptr, g.dsc);
        launch_check("k_split_scan");
        if (L <= LEAVES_SMALL) k_root_select<LEAVES_SMALL><<<1, 512, 0, stream>>>(g);
        else k_root_select<GROW_MAX_LEAVES><<<1, 512, 0, stream>>>(g);
        launch_check("k_root_select");
        // split steps: each is a no-op once the tree is complete; each commits at least one split
        uint32_t s = 0, batch = std::max<uint32_t>(2, last_steps ? last_steps : 8);
        const uint32_t max_steps = L;
        for (;;) {
            const uint32_t end = std::min(max_steps, s + batch);
            for (; s < end; ++s) {
                const uint32_t parity = s & 1u;
                hipEvent_t e0 = nullptr, e1 = nullptr;
                if (prof.on) {
                    e0 = event();
                    e1 = event();
                    hip_check(hipEventRecord(e0, stream), "event");
                }
                // the first slab's launch partitions; the others histogram the built children, consecutive slabs
                // of one kernel in one launch (k1 workgroups a slab)
                uint32_t launches = 0;
                for (size_t si = 0; si < slabs.size();) {
                    size_t sj = si + 1;
                    if (si > 0)
                        while (sj < slabs.size() && slabs[sj].same_launch(slabs[si])) ++sj;
                    const Slab &sl = slabs[si];
                    StepArgs sa{slab_bins.p + sl.bins_off, slab_stride(sl), step_partial.p + 2 * sl.step_partial_off, d_fmt.p + si * k1_groups(),
                                slab_col_bins.p + sl.col_bins_off, slab_pos_word.p + sl.pos_off, sl.row_bytes() / 4, k1_groups(), packed.p,
                                train.col.p, col16, rows, part.p, part2.p, tile_status.p, d_plans.p + parity, g.ctl, flush_rows(),
                                si == 0 ? 1u : 0u, g.tile_cap, codes ? codes0.p : nullptr, codes ? codes1.p : nullptr};
                    // a launch of one slab stops at the workgroups a step of jcap jobs can use (the plan's rounding
                    // takes at most one more a job); one of several slabs takes k1 a slab
                    const uint32_t grid = sj - si == 1 ? step_target + g.jcap : k1_groups() * static_cast<uint32_t>(sj - si);
                    // the instance with carried gradient codes when the units fit them (never with separate counters)
#define SROCM_STEP_CASE(id, W, WIDE, PACK, DP)                                                                    \
    case id:                                                                                                      \
        if (codes) k_step_rows<W, WIDE, PACK, false, DP, true><<<grid, 1024, 0, stream>>>(sa);                    \
        else k_step_rows<W, WIDE, PACK, false, DP, false><<<grid, 1024, 0, stream>>>(sa);                         \
        break;
                    switch (slabs[si].kernel()) {
                    SROCM_STEP_CASE(32, 32, false, 1, 0)
                    SROCM_STEP_CASE(64, 64, false, 1, 0)
                    SROCM_STEP_CASE(128, 128, false, 1, 0)
                    SROCM_STEP_CASE(33, 32, true, 1, 0)
                    SROCM_STEP_CASE(65, 64, true, 1, 0)
                    SROCM_STEP_CASE(129, 128, true, 1, 0)
                    SROCM_STEP_CASE(36, 32, false, 4, 0)
                    SROCM_STEP_CASE(68, 64, false, 4, 0)
                    SROCM_STEP_CASE(34, 32, false, 2, 0)
                    SROCM_STEP_CASE(66, 64, false, 2, 0)
                    SROCM_STEP_CASE(130, 128, false, 2, 0)
                    SROCM_STEP_CASE(3004, 128, false, 1, 4)
                    SROCM_STEP_CASE(3008, 128, false, 1, 8)
#undef SROCM_STEP_CASE
                    case 1032: k_step_rows<32, false, 1, true><<<grid, 1024, 0, stream>>>(sa); break;
                    case 1064: k_step_rows<64, false, 1, true><<<grid, 1024, 0, stream>>>(sa); break;
                    case 1033: k_step_rows<32, true, 1, true><<<grid, 1024, 0, stream>>>(sa); break;
                    case 1065: k_step_rows<64, true, 1, true><<<grid, 1024, 0, stream>>>(sa); break;
                    default: throw std::logic_error("no split-step kernel for the slab");
                    }
                    launch_check("k_step_rows");
                    ++launches;
                    si = sj;
                }
                if (prof.on) {
                    hip_check(hipEventRecord(e1, stream), "event");
                    prof.step_events.emplace_back(e0, e1);
                    prof.step_launches += static_cast<double>(launches);
                    sector_model(parity);
                }
                ReduceStepArgs ra{step_partial.p, d_fmt.p, d_cgs.p, d_plans.p + parity, slab_slot_flat.p};
                k_step_reduce<<<reduce_blocks(), 256, 0, stream>>>(g, ra);
                launch_check("k_step_reduce");
                ScanStepArgs sca{unit_feat.p, unit_segl.p, nseg_units, cat_feats.p, ncat, d_plans.p + parity};
                if (has_narrow64) k_step_scan<false><<<scan_blocks(), 256, 0, stream>>>(g, sca);
                if (has_seg_units) k_step_scan_seg<<<scan_blocks(), 256, 0, stream>>>(g, sca);
                if (has_wide) k_step_scan<true><<<scan_blocks(), 256, 0, stream>>>(g, sca);
                launch_check("k_step_scan");
                if (ncat) {
                    k_step_cat<<<std::min<uint32_t>(cus * 2, div_up(static_cast<uint64_t>(JMAX) * 2 * ncat, 4)), 256, 0, stream>>>(g, sca);
                    launch_check("k_step_cat");
                }
                SelectArgs sa2{fin_counts.p, d_plans.p + parity, d_plans.p + (parity ^ 1u)};
                if (L <= LEAVES_SMALL) k_step_select<LEAVES_SMALL><<<g.jcap, 512, 0, stream>>>(g, sa2);
                else k_step_select<GROW_MAX_LEAVES><<<g.jcap, 512, 0, stream>>>(g, sa2);
                launch_check("k_step_select");
            }
            if (after_steps) {
                // the readback goes on its own stream once the steps end, so the kernels queued after the steps do
                // not wait for the copy and the host takes the tree while they run (none of them writes the tree
                // block, except k_tree_nodes' error flag for a malformed tree, which the host learns of anyway)
                if (!tree_event) hip_check(hipEventCreateWithFlags(&tree_event, hipEventDisableTiming), "hipEventCreate");
                if (!steps_event) hip_check(hipEventCreateWithFlags(&steps_event, hipEventDisableTiming), "hipEventCreate");
                hip_check(hipEventRecord(steps_event, stream), "event");
                hip_check(hipStreamWaitEvent(copy_stream, steps_event, 0), "stream wait");
                hip_check(hipMemcpyAsync(hb, dtree.p, lay.bytes, hipMemcpyDeviceToHost, copy_stream), "read tree");
                hip_check(hipEventRecord(tree_event, copy_stream), "event");
                (*after_steps)(g);
                hip_check(hipEventSynchronize(tree_event), "event synchronize");
                hc = *reinterpret_cast<const GrowCtl *>(hb + lay.ctl);
            } else {
                hc = read_ctl();
            }
            if (hc.done) break;
            if (s >= max_steps) fail(SROCM_ERR_INTERNAL, "the device learner did not finish the tree");
            batch = 2;
        }
        last_steps = hc.steps;
    } else {
        hc = read_ctl();
    }
    if (hc.error == 1) {
        const uint32_t *e = hc.err_info;
        fail(SROCM_ERR_INTERNAL, "a split sent no rows to one side (step job " + std::to_string(e[0]) + ", leaf " +
                                     std::to_string(e[1]) + ", " + std::to_string(e[3]) + " of " + std::to_string(e[2]) +
                                     " rows left, " + std::to_string(e[4]) + " tiles on " + std::to_string(e[5]) +
                                     (e[6] ? " workgroups, packed)" : " workgroups)"));
    }
    if (hc.error == 3) fail(SROCM_ERR_INTERNAL, "a partition tile waited too long for an earlier tile's count");
    if (hc.error == 6) fail(SROCM_ERR_INTERNAL, "malformed device tree");
    if (hc.error) fail(SROCM_ERR_INTERNAL, "device learner error " + std::to_string(hc.error));
    const uint32_t n = hc.num_leaves, ni = n - 1, ntent = hc.ntent;
    auto *iv = reinterpret_cast<const double *>(hb + lay.iv);
    auto *iw = reinterpret_cast<const double *>(hb + lay.iw);
    auto *lv = reinterpret_cast<const double *>(hb + lay.lv);
    auto *lw = reinterpret_cast<const double *>(hb + lay.lw);
    auto *ic = reinterpret_cast<const int64_t *>(hb + lay.ic);
    auto *lcn = reinterpret_cast<const int64_t *>(hb + lay.lc);
    auto *lt = reinterpret_cast<const int32_t *>(hb + lay.leaf_t);
    auto *sf = reinterpret_cast<const int32_t *>(hb + lay.sf);
    auto *lc = reinterpret_cast<const int32_t *>(hb + lay.lch);
    auto *rc = reinterpret_cast<const int32_t *>(hb + lay.rch);
    auto *lp = reinterpret_cast<const int32_t *>(hb + lay.lp);
    auto *ld = reinterpret_cast<const int32_t *>(hb + lay.ld);
    auto *tb = reinterpret_cast<const uint32_t *>(hb + lay.tb);
    auto *sgn = reinterpret_cast<const float *>(hb + lay.sg);
    auto *lb = reinterpret_cast<const uint32_t *>(hb + lay.lb);
    auto *dl = reinterpret_cast<const uint8_t *>(hb + lay.dl);
    auto *lrg = reinterpret_cast<const uint32_t *>(hb + lay.lr);
    tree = HostTree{};
    tree.num_leaves = n;
    tree.split_feature.assign(sf, sf + ni);
    tree.left_child.assign(lc, lc + ni);
    tree.right_child.assign(rc, rc + ni);
    tree.threshold_bin.assign(tb, tb + ni);
    tree.default_left.assign(dl, dl + ni);
    tree.split_gain.assign(sgn, sgn + ni);
    tree.internal_value.assign(iv, iv + ni);
    tree.internal_weight.assign(iw, iw + ni);
    tree.internal_count.assign(ic, ic + ni);
    tree.leaf_value.assign(lv, lv + n);
    tree.leaf_weight.assign(lw, lw + n);
    tree.leaf_count.assign(lcn, lcn + n);
    tree.leaf_parent.assign(lp, lp + n);
    tree.leaf_depth.assign(ld, ld + n);
    tree.left_bins.assign(lb, lb + static_cast<size_t>(ni) * 8);
    leaves.assign(n, GrowLeaf{});
    for (uint32_t i = 0; i < n; ++i) {
        const int32_t k = lt[i];
        if (k < 0 || static_cast<uint32_t>(k) >= ntent) fail(SROCM_ERR_INTERNAL, "device learner lost a leaf");
        leaves[i].range = srocm_leaf_range{lrg[2 * i], lrg[2 * i + 1]};
    }
    splits.assign(ni, srocm_bin_split{});
    for (uint32_t k = 0; k < ni; ++k) {  // learner.rs:432-452, as the device planned each split
        const srocm_feature &m = feats[tree.split_feature[k]];
        srocm_bin_split &bs = splits[k];
        std::copy(lb + 8 * static_cast<size_t>(k), lb + 8 * static_cast<size_t>(k) + 8, bs.left_bins);
        bs.group = m.group;
        bs.column = m.column;
    }

    // the final row order: now, or (the boosting loop's last tree) when a call next reads the partition
    if (final_order && root_searched) {
        if (defer_order) pending_order = PendingOrder{true, n, ntent, std::vector<int32_t>(lt, lt + n)};
        else restore_order(n, ntent, lt);
    }
    if (prof.on && root_searched) {  // the root histogram was counted by launch_hist
        prof.builds += hc.hist_builds;
        prof.rows += hc.hist_rows;
        prof.bins += hc.hist_bins;
        prof.part_rows += hc.part_rows;
        // partition: 4 B row id read, the split's bin (1 B, 2 B with two-byte groups), 4 B row id write per parent
        // row; histogram: the built child's used bins and 4 B packed gradients per row
        prof.step_bytes += (col16 ? 10.0 : 9.0) * hc.part_rows + hc.hist_bins * (col16 ? 2.0 : 1.0) + 4.0 * hc.hist_rows;
        prof.expansions += hc.expansions;
        prof.splits += static_cast<double>(ni);
        prof.steps += hc.steps;
    }
}

// boosting.rs:100-108 and objective/mod.rs:92-109
double Context::boost_init(const srocm_train_params &p) {
    require_loaded();
    double score = 0.0;
    if (p.boost_from_average && objective != SROCM_OBJ_LAMBDARANK) {
        double sum_label = 0.0, sum_weight = 0.0;
        const float *lab = h_label_v.data();
        if (objective == SROCM_OBJ_BINARY) {  // binary.rs:11-25
            if (has_weight) {
                for (uint64_t i = 0; i < rows; ++i) {
                    float pos = lab[i] > 0.0f ? 1.0f : 0.0f;
                    sum_label = sum_label + static_cast<double>(pos * h_weight_v[i]);
                    sum_weight = sum_weight + static_cast<double>(h_weight_v[i]);
                }
            } else {
                for (uint64_t i = 0; i < rows; ++i) sum_label += lab[i] > 0.0f ? 1.0 : 0.0;
                sum_weight = static_cast<double>(rows);
            }
            double pr = std::clamp(sum_label / sum_weight, K_EPS_H, 1.0 - K_EPS_H);
            score = std::log(pr / (1.0 - pr)) / p.sigmoid;
        } else {  // regression.rs:60-67
            if (has_weight) {
                for (uint64_t i = 0; i < rows; ++i) {
                    sum_label = sum_label + static_cast<double>(lab[i] * h_weight_v[i]);
                    sum_weight = sum_weight + static_cast<double>(h_weight_v[i]);
                }
            } else {
                for (uint64_t i = 0; i < rows; ++i) sum_label += static_cast<double>(lab[i]);
                sum_weight = static_cast<double>(rows);
            }
            score = sum_label / sum_weight;
        }
        score = std::fabs(score) > K_EPS_H ? score : 0.0;
    }
    for (uint32_t d = 0; d <= valid.size(); ++d) init_scores(d, score);
    sync();
    init_score_value = score;
    trees_added = 0;
    return score;
}

// split.rs:966-985 feature_mask
static void feature_mask(const std::vector<srocm_feature> &feats, double fraction, uint32_t seed, uint32_t iteration,
                         std::vector<uint8_t> &mask) {
    std::vector<uint32_t> usable;
    for (uint32_t f = 0; f < feats.size(); ++f)
        if (feats[f].num_bins) usable.push_back(f);
    mask.assign(feats.size(), 0);
    if (fraction >= 1.0) {
        for (uint32_t f : usable) mask[f] = 1;
        return;
    }
    size_t count = std::max<size_t>(static_cast<size_t>(sat_i64_h(static_cast<double>(usable.size()) * fraction + 0.5)),
                                    std::min<size_t>(usable.size(), 1));
    std::vector<std::pair<float, uint32_t>> keyed;
    for (uint32_t f : usable) keyed.emplace_back(uniform_h(seed, 3u, iteration, f), f);
    std::sort(keyed.begin(), keyed.end(), [](const auto &a, const auto &b) {
        int c = total_cmp_f(a.first, b.first);
        if (c != 0) return c < 0;
        return a.second < b.second;
    });
    for (size_t i = 0; i < count && i < keyed.size(); ++i) mask[keyed[i].second] = 1;
}

// The reference's row order after a grown tree (cpu.rs:556-599 keeps every leaf ascending), from the speculative
// leaves the tree's steps left on the device (d_tl, `ntent` of them) and `lt`, each of the `n` committed leaves'
// speculative leaf: each unexpanded speculative leaf's rows into the first buffer in ascending order, then each
// committed leaf whose expansion was dropped merged from its runs. Its buffers are sized by ensure_grow, so it
// allocates nothing.
void Context::restore_order(uint32_t n, uint32_t ntent, const int32_t *lt) {
    // the final row order (cpu.rs:556-599 keeps every leaf ascending): each unexpanded speculative leaf's rows into
    // the first buffer in ascending order, then each leaf whose expansion was dropped merged from its runs
    const TLeaf *tl = reinterpret_cast<const TLeaf *>(h_result.p);
    hip_check(hipMemcpyAsync(h_result.p, d_tl.p, static_cast<size_t>(ntent) * sizeof(TLeaf), hipMemcpyDeviceToHost, stream), "read leaves");
    sync();
    std::vector<RowRun> runs;
    for (uint32_t k = 0; k < ntent; ++k)
        if (tl[k].state == T_LEAF && tl[k].count && (tl[k].buf || tl[k].rev))
            runs.push_back(RowRun{tl[k].begin, tl[k].count, tl[k].buf, tl[k].rev});
    std::vector<MergeJob> merges;
    std::vector<uint32_t> starts;
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t k = static_cast<uint32_t>(lt[i]);
        if (tl[k].state != T_EXPANDED) continue;
        MergeJob m{tl[k].begin, tl[k].count, static_cast<uint32_t>(starts.size()), 0};
        std::vector<uint32_t> stack{k};  // the unexpanded leaves below k, in row order (left child first)
        while (!stack.empty()) {
            const uint32_t x = stack.back();
            stack.pop_back();
            if (x >= ntent) fail(SROCM_ERR_INTERNAL, "device learner lost a leaf");
            if (tl[x].state == T_EXPANDED) {
                stack.push_back(static_cast<uint32_t>(tl[x].kid) + 1);
                stack.push_back(static_cast<uint32_t>(tl[x].kid));
            } else if (tl[x].count) {
                starts.push_back(tl[x].begin - m.begin);
                ++m.runs;
            }
        }
        starts.push_back(m.count);
        if (m.runs > 1) merges.push_back(m);
        else starts.resize(m.first);
    }
    if (!runs.empty() || !merges.empty()) {
        const size_t rb = runs.size() * sizeof(RowRun), mb = merges.size() * sizeof(MergeJob), sb = starts.size() * 4;
        h_fix.alloc(rb + mb + sb + 64);
        std::memcpy(h_fix.p, runs.data(), rb);
        std::memcpy(h_fix.p + rb, merges.data(), mb);
        std::memcpy(h_fix.p + rb + mb, starts.data(), sb);
        uint32_t longest = 1;
        if (!runs.empty()) {
            d_runs.alloc(runs.size());
            hip_check(hipMemcpyAsync(d_runs.p, h_fix.p, rb, hipMemcpyHostToDevice, stream), "upload runs");
            for (const RowRun &r : runs) longest = std::max(longest, r.count);
            k_consolidate<<<dim3(std::min<uint32_t>(div_up(longest, 256 * 4), 64), static_cast<uint32_t>(runs.size())), 256, 0, stream>>>(
                d_runs.p, part2.p, part.p);
            launch_check("k_consolidate");
        }
        if (!merges.empty()) {
            d_merges.alloc(merges.size());
            d_starts.alloc(starts.size());
            hip_check(hipMemcpyAsync(d_merges.p, h_fix.p + rb, mb, hipMemcpyHostToDevice, stream), "upload merges");
            hip_check(hipMemcpyAsync(d_starts.p, h_fix.p + rb + mb, sb, hipMemcpyHostToDevice, stream), "upload merges");
            longest = 1;
            uint32_t most = 1;
            for (const MergeJob &m : merges) {
                longest = std::max(longest, m.count);
                most = std::max(most, m.runs);
            }
            dim3 grid(std::min<uint32_t>(div_up(longest, 256 * 4), 256), static_cast<uint32_t>(merges.size()));
            // pairwise rounds between the two buffers, every leaf's rows moved in each; an odd count leaves the
            // result in the second buffer
            uint32_t rounds = 0;
            while ((1u << rounds) < most) ++rounds;
            for (uint32_t t = 0; t < rounds; ++t) {
                const bool even = (t & 1u) == 0;
                k_merge_round<<<grid, 256, 0, stream>>>(d_merges.p, d_starts.p, t, even ? part.p : part2.p, even ? part2.p : part.p);
                launch_check("k_merge_round");
            }
            if (rounds & 1u) {
                k_copy_back<<<grid, 256, 0, stream>>>(d_merges.p, part2.p, part.p);
                launch_check("k_copy_back");
            }
        }
    }
}

// boosting.rs:227-324 train_one_iter / add, `count` times
uint32_t Context::boost(const srocm_train_params &p, uint32_t first, uint32_t count, srocm_grown_tree *trees) {
    require_loaded();
    bool constant_hessian = objective == SROCM_OBJ_REGRESSION && !has_weight;  // objective/mod.rs:84-89
    check_quant_units(p.num_grad_quant_bins / 2, p.num_grad_quant_bins);
    set_mode(q32_for(p.num_grad_quant_bins / 2, p.num_grad_quant_bins), p.num_grad_quant_bins);
    uint32_t done = 0;
    HostTree tree;
    std::vector<srocm_bin_split> splits;
    std::vector<GrowLeaf> leaves;
    std::vector<uint8_t> mask;
    // A renewed tree's leaf values are made on the device, in the tree's own slot of d_leaf_vw, and come back with
    // every other tree's of the call in one copy at its end (a copy after each tree idled the GPU between
    // iterations); the trees' copies into `trees` wait for them.
    struct Pending {
        HostTree tree;
        std::vector<GrowLeaf> leaves;
        uint32_t index = 0;  // the tree's index in the call, and its slot
    };
    std::vector<Pending> pends;
    const size_t VW = 2 * static_cast<size_t>(GROW_MAX_LEAVES) + 1;
    if (p.quant_train_renew_leaf != 0) d_leaf_vw.alloc(static_cast<size_t>(count) * VW);
    auto finalize = [&]() {
        if (pends.empty()) return;
        const size_t n = (static_cast<size_t>(pends.back().index) + 1) * VW;
        h_leaf_vw.alloc(n);
        hip_check(hipMemcpyAsync(h_leaf_vw.p, d_leaf_vw.p, n * sizeof(double), hipMemcpyDeviceToHost, stream), "read leaf values");
        sync();
        for (Pending &pd : pends) {
            const uint32_t nl = pd.tree.num_leaves;
            const double *vw = h_leaf_vw.p + static_cast<size_t>(pd.index) * VW;
            // the leaves k_tree_nodes let through (after the tree's readback, so checked here)
            if (vw[2 * GROW_MAX_LEAVES] != static_cast<double>(nl)) fail(SROCM_ERR_INTERNAL, "malformed device tree");
            for (uint32_t l = 0; l < nl; ++l) {
                pd.tree.leaf_value[l] = vw[l];
                pd.tree.leaf_weight[l] = vw[GROW_MAX_LEAVES + l];
            }
            if (trees) copy_tree(pd.tree, pd.leaves, &trees[pd.index]);
        }
        pends.clear();
    };
    for (uint32_t it = first; it < first + count; ++it) {
        // lambdarank: an iteration whose device factors were flagged is taken again with the host's (the flag also
        // closed its leaf-renewal gate, so nothing of it reached the scores)
        bool host_factors = false;
    again:
        // quantize.rs:56-84 on the device: nothing waits for the gradient maxima
        launch_gradients(host_factors);
        d_scales.alloc(1);
        k_quant_spec<<<1, MAX_SLOTS, 0, stream>>>(maxima.p, d_scales.p, p.num_grad_quant_bins, constant_hessian ? 1u : 0u, 1.0,
                                           p.stochastic_rounding != 0 ? 1u : 0u, p.data_random_seed, it);
        launch_check("k_quant_spec");
        maxima_clear = true;
        if (rows) {
            k_quantize_dev<<<grid_rows(rows), 256, 0, stream>>>(grad.p, hess.p, packed.p, rows, row_offset, d_scales.p);
            launch_check("k_quantize");
        }
        queue_rank_flag();
        max_gq = static_cast<int64_t>(p.num_grad_quant_bins / 2);
        max_hq = static_cast<int64_t>(p.num_grad_quant_bins);
        quantized_once = true;
        const bool bias = trees_added == 0 && init_score_value != 0.0;
        const bool renew = p.quant_train_renew_leaf != 0;
        srocm_bag bag{};
        if (p.bagging_fraction < 1.0 && p.bagging_freq > 0) {
            bag.kind = SROCM_BAG_BERNOULLI;
            bag.seed = p.bagging_seed;
            bag.round = it / p.bagging_freq;
            bag.fraction = p.bagging_fraction;
        }
        uint32_t local_rows = reset_partition(bag);
        feature_mask(feats, p.feature_fraction, p.feature_fraction_seed, it, mask);
        srocm_grow_spec gs{};
        gs.cfg = p.cfg;
        gs.num_leaves = p.num_leaves;
        gs.max_depth = p.max_depth;
        gs.grad_scale = 1.0;  // unused: GrowState takes d_scales
        gs.hess_scale = 1.0;
        gs.feature_mask = mask.data();
        gs.root = srocm_leaf_range{0, local_rows};
        gs.root_count = local_rows;
        const bool last = it + 1 == first + count;
        // learner.rs:376-404 on the device, queued behind each batch of the tree's steps and gated there by the tree
        // being complete with a split: the rows' leaves from one walk give the sums; k_leaf_values makes the shrunk
        // (and, for the first tree, biased) leaf values; the scores take them; the values go to the host
        const std::function<void(const GrowState &)> renew_on_device = [&](const GrowState &gst) {
            const size_t L = GROW_MAX_LEAVES;
            d_nodes.alloc(L);
            d_leaf_out.alloc(2 * L);
            d_leaf_values.alloc(L);
            double *dvw = d_leaf_vw.p + static_cast<size_t>(done) * VW;  // this tree's slot (an iteration taken
                                                                          // again writes it again)
            d_gate.alloc(1);
            leaf_of.alloc(rows);
            k_tree_nodes<<<1, 512, 0, stream>>>(gst, d_nodes.p, d_leaf_out.p, d_gate.p, dvw + 2 * L,
                                                rank_flag_pending ? d_rank_flag.p : nullptr);
            launch_check("k_tree_nodes");
            TreeLeavesArgs a{};
            a.colbins = train.col.p;
            a.col16 = col16;
            a.rows = rows;
            a.nodes = d_nodes.p;
            a.leaf_of = leaf_of.p;
            a.grad = grad.p;
            a.hess = hess.p;
            a.dsc = d_scales.p;
            a.sums = d_leaf_out.p;
            a.bag = bag.kind == SROCM_BAG_BERNOULLI ? 1u : 0u;
            a.bag_seed = bag.seed;
            a.bag_round = bag.round;
            a.row_offset = row_offset;
            a.fraction = bag.fraction;
            a.gate = d_gate.p;
            launch_tree_leaves(a, p.num_leaves);
            LeafValueArgs la{d_leaf_out.p, d_gate.p, d_scales.p, 0u, bias ? 1u : 0u, 1.0f, 1.0f, p.cfg.lambda_l1, p.cfg.lambda_l2,
                             p.learning_rate, init_score_value, dvw, dvw + L, d_leaf_values.p};
            k_leaf_values<<<1, 512, 0, stream>>>(la);
            launch_check("k_leaf_values");
            if (train.rows)
                k_add_leaf_values<<<grid_rows(train.rows), 256, 0, stream>>>(leaf_of.p, d_leaf_values.p, train.scores.p, train.rows, d_gate.p);
            for (auto &v : valid)
                if (v.rows) k_add_tree<<<grid_rows(v.rows), 256, 0, stream>>>(v.col.p, col16, v.rows, d_nodes.p, d_leaf_values.p, v.scores.p, d_gate.p);
            launch_check("k_add_tree");
        };
        struct ScalesFromDevice {  // GrowState takes the device's scales while this tree grows
            const DevScales *&slot;
            ScalesFromDevice(const DevScales *&s, const DevScales *v) : slot(s) { slot = v; }
            ~ScalesFromDevice() { slot = nullptr; }
        } from_device(grow_dsc, d_scales.p);
        // the last tree's row order waits for the first call that reads the partition
        struct Defer {
            bool &flag;
            Defer(bool &f, bool on) : flag(f) { flag = on; }
            ~Defer() { flag = false; }
        } defer(defer_order, last);
        grow(gs, tree, splits, leaves, last, renew ? &renew_on_device : nullptr);
        if (!host_factors && rank_factors_vetoed()) {
            host_factors = true;
            goto again;
        }
        if (tree.num_leaves == 1) {  // boosting.rs:301-310
            if (trees_added == 0) {
                HostTree c;
                c.leaf_value[0] = init_score_value;
                if (trees) copy_tree(c, {}, &trees[done]);
                ++done;
                ++trees_added;
            }
            break;
        }
        if (renew) {
            // the scores and leaf values were queued behind the tree's steps (renew_on_device); the values reach
            // the host at the end of the call
            tree.shrink(p.learning_rate);  // the internal values (the leaf values are replaced on arrival)
            if (bias) tree.add_bias(init_score_value);
            pends.push_back(Pending{tree, leaves, done});
            ++done;
            ++trees_added;
            continue;
        }
        std::vector<srocm_device_node> nodes(splits.size());
        for (size_t k = 0; k < nodes.size(); ++k) {
            nodes[k].split = splits[k];
            nodes[k].left = tree.left_child[k];
            nodes[k].right = tree.right_child[k];
        }
        const uint32_t nn = static_cast<uint32_t>(nodes.size()), nl = tree.num_leaves;
        upload_nodes(nodes.data(), nn, nl);
        // boosting.rs:313-324
        tree.shrink(p.learning_rate);
        std::vector<float> lv(tree.leaf_value.size());
        for (size_t i = 0; i < lv.size(); ++i) lv[i] = static_cast<float>(tree.leaf_value[i]);
        if (bias) {
            tree.add_bias(init_score_value);
            for (size_t i = 0; i < lv.size(); ++i) lv[i] = static_cast<float>(tree.leaf_value[i] - init_score_value);  // replay.rs:38-40
        }
        upload_leaf_values(lv.data(), nl);
        apply_tree(train, nn, lv[0], p.quant_train_renew_leaf != 0);
        for (auto &v : valid) apply_tree(v, nn, lv[0], false);
        if (trees) copy_tree(tree, leaves, &trees[done]);
        ++done;
        ++trees_added;
    }
    finalize();
    return done;
}

// ---------------------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------------------

thread_local std::string g_create_error;

template <typename F>
int guard(void *ctx, F &&body) {
    Context *c = static_cast<Context *>(ctx);
    if (!c) return SROCM_ERR_DEVICE;
    try {
        body(*c);
        c->error.clear();
        return SROCM_OK;
    } catch (const Failure &f) {
        c->error = f.what();
        return f.kind;
    } catch (const std::bad_alloc &) {
        c->error = "host out of memory";
        return SROCM_ERR_DEVICE;
    } catch (const std::exception &e) {
        c->error = e.what();
        return SROCM_ERR_INTERNAL;
    }
}

}  // namespace

extern "C" {

int srocm_is_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    for (int i = 0; i < n; ++i) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, i) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) return 1;
    }
    return 0;
}

int srocm_create(int ordinal, void **out) {
    if (!out) return SROCM_ERR_DEVICE;
    *out = nullptr;
    try {
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        if (e != hipSuccess || n <= 0) fail(SROCM_ERR_DEVICE, "rocm: no HIP device is available");
        int dev = ordinal < 0 ? 0 : ordinal;
        if (dev >= n) fail(SROCM_ERR_DEVICE, "rocm: device " + std::to_string(dev) + " of " + std::to_string(n));
        hipDeviceProp_t prop;
        hip_check(hipGetDeviceProperties(&prop, dev), "device properties");
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            fail(SROCM_ERR_DEVICE, std::string("rocm: device is ") + prop.gcnArchName + ", this build targets gfx950");
        hip_check(hipSetDevice(dev), "set device");
        auto c = std::make_unique<Context>();
        c->device = dev;
        c->cus = static_cast<uint32_t>(prop.multiProcessorCount);
        c->device_name = prop.name[0] ? prop.name : prop.gcnArchName;  // the name can be empty; the architecture is not
        c->scratch_at = scratch_address(dev);
        hip_check(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "create stream");
        hip_check(hipStreamCreateWithFlags(&c->copy_stream, hipStreamNonBlocking), "create stream");
        c->h_u32.alloc(2 * MAX_SLOTS);
        *out = c.release();
        g_create_error.clear();
        return SROCM_OK;
    } catch (const Failure &f) {
        g_create_error = f.what();
        return f.kind;
    } catch (const std::exception &e) {
        g_create_error = e.what();
        return SROCM_ERR_INTERNAL;
    }
}

void srocm_destroy(void *ctx) {
    Context *c = static_cast<Context *>(ctx);
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    delete c;
}

const char *srocm_last_error(const void *ctx) {
    if (!ctx) return g_create_error.c_str();
    return static_cast<const Context *>(ctx)->error.c_str();
}

int srocm_name(void *ctx, char *buf, size_t len) {
    return guard(ctx, [&](Context &c) {
        std::string n = c.device_name + " (rocm, " + std::to_string(c.cus) + " CUs)";
        if (buf && len) {
            std::strncpy(buf, n.c_str(), len - 1);
            buf[len - 1] = 0;
        }
    });
}

int srocm_slab_layout(void *ctx, uint32_t *out, uint32_t cap, uint32_t *count) {
    return guard(ctx, [&](Context &c) {
        c.require_loaded();
        for (size_t i = 0; i < c.slabs.size() && i < cap && out; ++i) {
            const Slab &s = c.slabs[i];
            out[4 * i] = s.width;
            out[4 * i + 1] = s.row_bytes();
            out[4 * i + 2] = s.dense_passes ? 0u : (s.wide ? 1u : s.pack);
            out[4 * i + 3] = (s.wide ? 1u : 0u) | (s.q32 ? 2u : 0u) | (s.dense_passes ? 4u : 0u);
        }
        if (count) *count = static_cast<uint32_t>(c.slabs.size());
    });
}

int srocm_load(void *ctx, const srocm_dataset *train, const srocm_dataset *const *valid, uint32_t num_valid,
               const srocm_objective *objective) {
    return guard(ctx, [&](Context &c) {
        hip_check(hipSetDevice(c.device), "set device");
        c.load(train, valid, num_valid, objective);
    });
}

int srocm_init_scores(void *ctx, uint32_t dataset, double value) {
    return guard(ctx, [&](Context &c) {
        c.init_scores(dataset, value);
        c.sync();
    });
}

int srocm_compute_gradients(void *ctx, double *max_abs_grad, double *max_hess) {
    return guard(ctx, [&](Context &c) {
        auto [g, h] = c.compute_gradients();
        c.sync();
        if (max_abs_grad) *max_abs_grad = g;
        if (max_hess) *max_hess = h;
    });
}

int srocm_set_gradients(void *ctx, const float *grad, const float *hess, uint64_t n, double *max_abs_grad, double *max_hess) {
    return guard(ctx, [&](Context &c) {
        auto [g, h] = c.set_gradients(grad, hess, n);
        if (max_abs_grad) *max_abs_grad = g;
        if (max_hess) *max_hess = h;
    });
}

int srocm_gradients(void *ctx, float *grad, float *hess, size_t len) {
    return guard(ctx, [&](Context &c) {
        c.require_loaded();
        if (len != c.rows) fail(SROCM_ERR_DEVICE, "gradient buffers of " + std::to_string(len) + " values, expected " + std::to_string(c.rows));
        if (len) {
            hip_check(hipMemcpyAsync(grad, c.grad.p, len * 4, hipMemcpyDeviceToHost, c.stream), "read grad");
            hip_check(hipMemcpyAsync(hess, c.hess.p, len * 4, hipMemcpyDeviceToHost, c.stream), "read hess");
        }
        c.sync();
    });
}

int srocm_partition_rows(void *ctx, uint32_t *out, size_t len) {
    return guard(ctx, [&](Context &c) {
        c.require_loaded();
        if (len > c.rows) fail(SROCM_ERR_DEVICE, "partition read of " + std::to_string(len) + " rows, the training set has " + std::to_string(c.rows));
        if (len && !out) fail(SROCM_ERR_DEVICE, "null output");
        c.ensure_order();
        if (len) hip_check(hipMemcpyAsync(out, c.part.p, len * 4, hipMemcpyDeviceToHost, c.stream), "read partition");
        c.sync();
    });
}

int srocm_quantize(void *ctx, const srocm_quant_spec *spec) {
    return guard(ctx, [&](Context &c) {
        if (!spec) fail(SROCM_ERR_DEVICE, "null quantization spec");
        c.quantize(*spec);
        c.sync();
    });
}

int srocm_reset_partition(void *ctx, const srocm_bag *bag, uint32_t *count) {
    return guard(ctx, [&](Context &c) {
        srocm_bag all{};
        uint32_t n = c.reset_partition(bag ? *bag : all);
        c.sync();
        if (count) *count = n;
    });
}

int srocm_set_histogram_features(void *ctx, const uint8_t *used, uint32_t num_features) {
    return guard(ctx, [&](Context &c) {
        c.require_loaded();
        for (uint32_t f = 0; f < c.nf; ++f) c.used[f] = (!used || f >= num_features) ? 1 : used[f];
    });
}

int srocm_histogram(void *ctx, srocm_leaf_range leaf, int quantized, double *out, size_t len) {
    return guard(ctx, [&](Context &c) { c.histogram(leaf, quantized, out, len); });
}

int srocm_partition(void *ctx, srocm_leaf_range leaf, const srocm_bin_split *split, uint32_t *left) {
    return guard(ctx, [&](Context &c) {
        if (!split) fail(SROCM_ERR_DEVICE, "null split");
        uint32_t l = c.partition(leaf, *split);
        if (left) *left = l;
    });
}

int srocm_partition_and_histogram(void *ctx, srocm_leaf_range leaf, const srocm_bin_split *split, uint32_t side,
                                  int quantized, double *out, size_t len, uint32_t *left) {
    return guard(ctx, [&](Context &c) {
        if (!split) fail(SROCM_ERR_DEVICE, "null split");
        uint32_t l = c.partition_and_histogram(leaf, *split, side, quantized, out, len);
        if (left) *left = l;
    });
}

int srocm_leaf_sums(void *ctx, const srocm_leaf_range *leaves, uint32_t num_leaves, float grad_scale, float hess_scale,
                    int64_t *out) {
    return guard(ctx, [&](Context &c) { c.leaf_sums(leaves, num_leaves, grad_scale, hess_scale, out); });
}

int srocm_add_tree(void *ctx, const srocm_device_node *nodes, uint32_t num_nodes, const float *leaf_values,
                   uint32_t num_leaf_values) {
    return guard(ctx, [&](Context &c) { c.add_tree(nodes, num_nodes, leaf_values, num_leaf_values); });
}

int srocm_scores(void *ctx, uint32_t dataset, float *out, size_t len) {
    return guard(ctx, [&](Context &c) { c.scores(dataset, out, len); });
}

int srocm_find_best_split(void *ctx, const double *hist, size_t len, const srocm_feature *features,
                          uint32_t num_features, const uint8_t *evaluate, const srocm_sums *sums, double grad_scale,
                          double hess_scale, const srocm_split_config *cfg, srocm_split_info *out,
                          uint8_t *splittable) {
    return guard(ctx, [&](Context &c) {
        if ((!hist && len) || (!features && num_features) || (!evaluate && num_features) || !sums || !cfg || !out ||
            (!splittable && num_features))
            fail(SROCM_ERR_DEVICE, "null argument");
        c.find_best_split(hist, len, features, num_features, evaluate, *sums, grad_scale, hess_scale, *cfg, out, splittable);
    });
}

int srocm_hist_slots(void *ctx, uint32_t num_slots) {
    return guard(ctx, [&](Context &c) { c.hist_slots(num_slots); });
}

int srocm_histogram_slot(void *ctx, srocm_leaf_range leaf, uint32_t slot) {
    return guard(ctx, [&](Context &c) { c.histogram_slot(leaf, slot); });
}

int srocm_partition_and_histogram_slot(void *ctx, srocm_leaf_range leaf, const srocm_bin_split *split, uint32_t side,
                                       uint32_t slot, uint32_t *left) {
    return guard(ctx, [&](Context &c) {
        if (!split) fail(SROCM_ERR_DEVICE, "null split");
        uint32_t l = c.partition_and_histogram_slot(leaf, *split, side, slot);
        if (left) *left = l;
    });
}

int srocm_subtract(void *ctx, uint32_t parent_slot, uint32_t child_slot) {
    return guard(ctx, [&](Context &c) { c.subtract(parent_slot, child_slot); });
}

int srocm_read_slot(void *ctx, uint32_t slot, double *out, size_t len) {
    return guard(ctx, [&](Context &c) {
        if (!out && len) fail(SROCM_ERR_DEVICE, "null argument");
        c.read_slot(slot, out, len);
    });
}

int srocm_find_best_split_slot(void *ctx, uint32_t slot, const srocm_feature *features, uint32_t num_features,
                               const uint8_t *evaluate, const srocm_sums *sums, double grad_scale, double hess_scale,
                               const srocm_split_config *cfg, srocm_split_info *out, uint8_t *splittable) {
    return guard(ctx, [&](Context &c) {
        if ((!features && num_features) || (!evaluate && num_features) || !sums || !cfg || !out ||
            (!splittable && num_features))
            fail(SROCM_ERR_DEVICE, "null argument");
        c.find_best_split_slot(slot, features, num_features, evaluate, *sums, grad_scale, hess_scale, *cfg, out, splittable);
    });
}

int srocm_grow(void *ctx, const srocm_grow_spec *spec, srocm_grown_tree *out) {
    return guard(ctx, [&](Context &c) {
        if (!spec || !out || !spec->feature_mask) fail(SROCM_ERR_DEVICE, "null argument");
        HostTree tree;
        std::vector<srocm_bin_split> splits;
        std::vector<GrowLeaf> leaves;
        c.grow(*spec, tree, splits, leaves);
        c.copy_tree(tree, leaves, out);
    });
}

int srocm_boost_init(void *ctx, const srocm_train_params *params, double *init_score) {
    return guard(ctx, [&](Context &c) {
        if (!params) fail(SROCM_ERR_CONFIG, "null parameters");
        double s = c.boost_init(*params);
        if (init_score) *init_score = s;
    });
}

int srocm_boost(void *ctx, const srocm_train_params *params, uint32_t first_iteration, uint32_t count,
                srocm_grown_tree *trees, uint32_t *trained) {
    return guard(ctx, [&](Context &c) {
        if (!params) fail(SROCM_ERR_CONFIG, "null parameters");
        if (params->num_leaves < 2) fail(SROCM_ERR_CONFIG, "num_leaves must be at least 2");
        // the reference takes 2..=64 (config.rs:416-421); up to 32766 is an extension (a packed row word holds h_q
        // below 32768)
        if (params->num_grad_quant_bins < 2 || params->num_grad_quant_bins > 32766 || params->num_grad_quant_bins % 2)
            fail(SROCM_ERR_CONFIG, "num_grad_quant_bins must be even and in 2..=32766");
        uint32_t n = c.boost(*params, first_iteration, count, trees);
        if (trained) *trained = n;
    });
}

int srocm_histogram_noalloc(void *ctx, srocm_leaf_range leaf, int64_t *out, size_t len, int wait) {
    return guard(ctx, [&](Context &c) {
        hip_check(hipSetDevice(c.device), "set device");
        c.histogram_noalloc(leaf, out, len, wait);
    });
}

int srocm_profile(void *ctx, int enable) {
    return guard(ctx, [&](Context &c) { c.profile(enable); });
}

int srocm_profile_read(void *ctx, double *out, uint32_t len) {
    return guard(ctx, [&](Context &c) {
        c.settle_profile();
        const Profile &p = c.prof;
        double v[SROCM_PROFILE_VALUES] = {p.hist_launches, p.hist_ms, p.hist_bytes, p.step_launches, p.step_ms, p.step_bytes,
                                          p.builds, p.rows, p.bins, p.part_rows, p.part_launches, p.part_ms,
                                          p.steps, p.expansions, p.splits, p.sector[0], p.sector[1], p.sector[2],
                                          p.sector[3], p.sector[4], p.sector[5], p.sector[6], p.sector[7],
                                          p.sector[8], p.sector[9], p.rank_redos};
        if (out) std::copy(v, v + std::min<uint32_t>(len, SROCM_PROFILE_VALUES), out);
    });
}

}  // extern "C"
