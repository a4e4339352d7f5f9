// synth.cpp - seeded synthetic workloads shaped like the benchmark configurations, already binned.
//
// Rows come from silvic's counter hash (crates/silvic-core/src/quantize.rs:14-31), so any row of any
// configuration is a pure function of (seed, stream, row) and regenerates identically on any host. Values are
// binned by an equal-frequency binner over a sample (bounds at midpoints between sampled values, the last one
// +inf, NaN in its own last bin when the sample has NaN) and laid out as silvic's `layout` does
// (crates/silvic-core/src/data/build.rs:336-383): non-trivial features in order, a new group whenever the
// next feature would take the current one past 8192 bins, each group's row stride its feature count rounded
// up to 4. The binner is this project's own, not LightGBM's `BinMapper` (data/bin_mapper.rs); the oracle and
// the device always consume the same binned dataset, so the training path's parity does not depend on it.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <memory>
#include <thread>
#include <vector>

namespace {

inline uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

// A draw in (0, 1) with 24 bits, keyed by (seed, stream, row).
inline double unit(uint32_t seed, uint32_t stream, uint64_t row) {
    uint32_t row_hash = mix32(static_cast<uint32_t>(row) ^ mix32(static_cast<uint32_t>(row >> 32)));
    uint32_t h = mix32(seed ^ mix32(stream ^ mix32(0x5eedu ^ row_hash)));
    return (static_cast<double>(h >> 8) + 0.5) * (1.0 / 16777216.0);
}

inline double normal(uint32_t seed, uint32_t stream, uint64_t row) {
    double u1 = unit(seed, 2 * stream, row), u2 = unit(seed, 2 * stream + 1, row);
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

constexpr uint32_t NAN_STREAM = 1u << 20;
constexpr uint32_t AUX_STREAM = 1u << 21;
constexpr uint32_t LABEL_STREAM = 1u << 22;
constexpr uint32_t QUERY_STREAM = 1u << 23;

struct Workload {
    uint32_t config = 0;
    uint64_t rows = 0;
    uint32_t cols = 0;
    uint32_t seed = 0;
    uint32_t max_bin = 255;
    uint32_t bin_bytes = 1;  // 2 when max_bin > 256
    // per input feature
    std::vector<uint32_t> num_bins, group, column, hist_offset, kind, nan_bin;
    std::vector<std::vector<double>> bounds;
    // per group
    std::vector<uint32_t> g_stride, g_hist_offset, g_total_bins;
    std::vector<std::vector<uint32_t>> g_features;
    std::vector<std::vector<uint8_t>> g_data;
    uint64_t total_bins = 0;
    std::vector<float> label;
    std::vector<uint32_t> query_boundaries;  // config 3: num_queries + 1
};

// Config 3's queries: Zipf-like sizes, floor(10 * u^(-1 / 0.35)) clipped to [10, 200] (a mean of about 100 rows),
// until the rows run out (the last query takes what is left).
std::vector<uint32_t> query_boundaries(uint32_t seed, uint64_t rows) {
    std::vector<uint32_t> b{0};
    uint64_t at = 0;
    for (uint64_t q = 0; at < rows; ++q) {
        const double size = std::floor(10.0 * std::pow(unit(seed, QUERY_STREAM, q), -1.0 / 0.35));
        const uint64_t n = std::min<uint64_t>(static_cast<uint64_t>(std::clamp(size, 10.0, 200.0)), rows - at);
        at += n;
        b.push_back(static_cast<uint32_t>(at));
    }
    return b;
}

// Raw value of feature j at row r (NaN for missing), per configuration.
double value(const Workload &w, uint32_t j, uint64_t r) {
    const uint32_t s = w.seed;
    switch (w.config) {
    case 1:  // 100k x 28 N(0,1)
        return normal(s, j, r);
    case 2: {  // 10M x 128: N(0,1) | lognormal(0,1) | integers [0,20); 10% NaN
        if (unit(s, NAN_STREAM + j, r) < 0.1) return std::numeric_limits<double>::quiet_NaN();
        if (j < w.cols / 2) return normal(s, j, r);
        if (j < 3 * w.cols / 4) return std::exp(normal(s, j, r));
        return std::floor(unit(s, 2 * j, r) * 20.0);
    }
    case 3:  // lambdarank docs: N(0,1) and exponential(1)
        return (j % 2 == 0) ? normal(s, j, r) : -std::log(unit(s, 2 * j, r));
    case 4: {  // 98% exact zeros; nonzeros exponential(1) or integers of cardinality 2..16
        if (unit(s, NAN_STREAM + j, r) < 0.98) return 0.0;
        uint32_t card = 2 + (mix32(j * 7919u + s) % 15);
        if (j % 2 == 0) return -std::log(unit(s, 2 * j, r));
        return 1.0 + std::floor(unit(s, 2 * j + 1, r) * card);
    }
    case 5:  // U[0,1)
        return unit(s, j, r);
    default:
        return 0.0;
    }
}

float label_of(const Workload &w, uint64_t r, const std::vector<double> &x) {
    const uint32_t s = w.seed;
    auto v = [&](uint32_t j) { return std::isnan(x[j]) ? 0.0 : x[j]; };
    switch (w.config) {
    case 1: {  // y = w.x + 0.5 sin(x0 x1) + N(0, 0.1), w ~ N(0,1) from seed 0
        double y = 0.0;
        for (uint32_t j = 0; j < w.cols; ++j) y += normal(0, AUX_STREAM + j, 0) * v(j);
        y += 0.5 * std::sin(v(0) * v(1)) + 0.1 * normal(s, LABEL_STREAM, r);
        return static_cast<float>(y);
    }
    case 2:
    case 4: {  // Bernoulli(sigmoid(sparse linear term over 16 features + 4 pairwise products))
        double z = 0.0;
        for (uint32_t i = 0; i < 16; ++i) {
            uint32_t j = (i * 37u + 3u) % w.cols;
            double scale = (w.config == 2 && j >= w.cols / 2 && j < 3 * w.cols / 4) ? 0.3 : 1.0;
            if (w.config == 2 && j >= 3 * w.cols / 4) scale = 0.1;
            z += normal(0, AUX_STREAM + i, 0) * scale * v(j);
        }
        for (uint32_t k = 0; k < 4; ++k) {
            uint32_t a = (k * 11u + 1u) % w.cols, b = (k * 29u + 7u) % w.cols;
            z += 0.5 * std::tanh(v(a)) * std::tanh(v(b));
        }
        double p = 1.0 / (1.0 + std::exp(-z));
        return unit(s, LABEL_STREAM, r) < p ? 1.0f : 0.0f;
    }
    case 3: {  // relevance 0..4 from a noisy monotone function of 8 features (4 normal, 4 exponential: mean 4)
        double z = -4.0;
        for (uint32_t i = 0; i < 8; ++i) z += v(i * 3);
        z += normal(s, LABEL_STREAM, r);
        return static_cast<float>(std::clamp(std::floor(z * 0.6 + 2.0), 0.0, 4.0));
    }
    case 5: {  // a piecewise-constant function of the features plus N(0, 0.05)
        double y = 0.0;
        for (uint32_t j = 0; j < 8; ++j) y += (x[j] > 0.5 ? 1.0 : 0.0) * (j + 1) + (x[j + 8] > 0.25 ? 0.5 : 0.0);
        return static_cast<float>(y + 0.05 * normal(s, LABEL_STREAM, r));
    }
    default:
        return 0.0f;
    }
}

template <typename F>
void parallel(uint64_t n, F fn) {
    unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> ts;
    uint64_t chunk = (n + threads - 1) / threads;
    for (unsigned t = 0; t < threads; ++t) {
        uint64_t b = t * chunk, e = std::min(n, b + chunk);
        if (b >= e) break;
        ts.emplace_back([=] { fn(b, e); });
    }
    for (auto &t : ts) t.join();
}

// Equal-frequency bounds over a sample; returns (bounds, nan_bin).
void find_bins(std::vector<double> sample, uint32_t max_bin, std::vector<double> &bounds, bool &nan_bin) {
    size_t nans = 0;
    std::vector<double> values;
    values.reserve(sample.size());
    for (double v : sample) {
        if (std::isnan(v)) ++nans;
        else values.push_back(v);
    }
    nan_bin = nans > 0;
    std::sort(values.begin(), values.end());
    bounds.clear();
    if (values.empty()) return;
    uint32_t numeric = nan_bin ? max_bin - 1 : max_bin;
    std::vector<double> distinct;
    for (double v : values)
        if (distinct.empty() || v != distinct.back()) distinct.push_back(v);
    if (distinct.size() <= numeric) {
        for (size_t i = 0; i + 1 < distinct.size(); ++i) bounds.push_back((distinct[i] + distinct[i + 1]) / 2.0);
    } else {
        size_t n = values.size();
        for (uint32_t k = 1; k < numeric; ++k) {
            double v = values[std::min(n - 1, (n * k) / numeric)];
            auto it = std::upper_bound(distinct.begin(), distinct.end(), v);
            if (it == distinct.end()) break;
            double b = (*(it - 1) + *it) / 2.0;
            if (bounds.empty() || b > bounds.back()) bounds.push_back(b);
        }
    }
    bounds.push_back(std::numeric_limits<double>::infinity());
}

inline uint32_t bin_of(const std::vector<double> &bounds, bool nan_bin, double v) {
    if (std::isnan(v)) {
        if (nan_bin) return static_cast<uint32_t>(bounds.size());
        v = 0.0;
    }
    return static_cast<uint32_t>(std::lower_bound(bounds.begin(), bounds.end(), v) - bounds.begin());
}

}  // namespace

extern "C" {

// Builds configuration `config` (1..5) with `rows` rows and `cols` features, binned with at most `max_bin`
// bins per feature (2..1024; above 256 the bins are stored as little-endian u16, two bytes per feature, the
// extension for max_bin > 255). Returns NULL for an unknown configuration or bad sizes.
void *synth_create(uint32_t config, uint64_t rows, uint32_t cols, uint32_t seed, uint32_t max_bin) {
    if (config < 1 || config > 5 || rows == 0 || cols == 0 || max_bin < 2 || max_bin > 1024) return nullptr;
    auto w = std::make_unique<Workload>();
    w->config = config;
    w->rows = rows;
    w->cols = cols;
    w->seed = seed;
    w->max_bin = max_bin;
    w->bin_bytes = max_bin > 256 ? 2u : 1u;
    // bin mappers from a sample of up to 200k rows (bin_construct_sample_cnt, config.rs:143)
    uint64_t sample_rows = std::min<uint64_t>(rows, 200000);
    uint64_t step = rows / sample_rows;
    w->bounds.resize(cols);
    std::vector<uint8_t> nan(cols);
    parallel(cols, [&](uint64_t b, uint64_t e) {
        for (uint64_t j = b; j < e; ++j) {
            std::vector<double> sample(sample_rows);
            for (uint64_t i = 0; i < sample_rows; ++i) sample[i] = value(*w, static_cast<uint32_t>(j), i * step);
            bool nb;
            find_bins(std::move(sample), max_bin, w->bounds[j], nb);
            nan[j] = nb;
        }
    });
    // layout (build.rs:336-383)
    uint32_t offset = 0;
    for (uint32_t j = 0; j < cols; ++j) {
        uint32_t nb = static_cast<uint32_t>(w->bounds[j].size()) + nan[j];
        bool trivial = nb <= 1;
        w->kind.push_back(trivial ? 0u : 1u);
        w->nan_bin.push_back(trivial ? 0u : nan[j]);
        w->num_bins.push_back(trivial ? 0u : nb);
        w->hist_offset.push_back(offset);
        if (trivial) {
            w->group.push_back(0);
            w->column.push_back(0);
            continue;
        }
        if (w->g_features.empty() || w->g_total_bins.back() + nb > 8192) {
            w->g_features.emplace_back();
            w->g_hist_offset.push_back(offset);
            w->g_total_bins.push_back(0);
        }
        w->group.push_back(static_cast<uint32_t>(w->g_features.size() - 1));
        w->column.push_back(static_cast<uint32_t>(w->g_features.back().size()) * w->bin_bytes);
        w->g_features.back().push_back(j);
        w->g_total_bins.back() += nb;
        offset += nb;
    }
    w->total_bins = offset;
    for (auto &f : w->g_features) w->g_stride.push_back(static_cast<uint32_t>((f.size() * w->bin_bytes + 3) / 4 * 4));
    w->g_data.resize(w->g_features.size());
    for (size_t g = 0; g < w->g_data.size(); ++g) w->g_data[g].assign(rows * w->g_stride[g], 0);
    w->label.resize(rows);
    if (config == 3) w->query_boundaries = query_boundaries(seed, rows);
    parallel(rows, [&](uint64_t b, uint64_t e) {
        std::vector<double> x(cols);
        for (uint64_t r = b; r < e; ++r) {
            for (uint32_t j = 0; j < cols; ++j) {
                x[j] = value(*w, j, r);
                if (w->num_bins[j] == 0) continue;
                uint32_t g = w->group[j];
                const uint32_t b = bin_of(w->bounds[j], w->nan_bin[j] != 0, x[j]);
                uint8_t *at = &w->g_data[g][r * w->g_stride[g] + w->column[j]];
                at[0] = static_cast<uint8_t>(b);
                if (w->bin_bytes == 2) at[1] = static_cast<uint8_t>(b >> 8);
            }
            w->label[r] = label_of(*w, r, x);
        }
    });
    return w.release();
}

void synth_free(void *h) { delete static_cast<Workload *>(h); }

// Per-feature metadata: num_bins, group, column, hist_offset, kind, nan_bin (6 x cols u32).
void synth_features(const void *h, uint32_t *out) {
    const Workload *w = static_cast<const Workload *>(h);
    for (uint32_t j = 0; j < w->cols; ++j) {
        uint32_t *o = out + 6 * j;
        o[0] = w->num_bins[j];
        o[1] = w->group[j];
        o[2] = w->column[j];
        o[3] = w->hist_offset[j];
        o[4] = w->kind[j];
        o[5] = w->nan_bin[j];
    }
}

uint32_t synth_num_groups(const void *h) { return static_cast<uint32_t>(static_cast<const Workload *>(h)->g_features.size()); }
uint64_t synth_total_bins(const void *h) { return static_cast<const Workload *>(h)->total_bins; }

// Group `g`: row stride, hist offset, total bins, feature count, bits per bin (8, or 16 above 256 bins).
void synth_group(const void *h, uint32_t g, uint32_t *out5) {
    const Workload *w = static_cast<const Workload *>(h);
    out5[0] = w->g_stride[g];
    out5[1] = w->g_hist_offset[g];
    out5[2] = w->g_total_bins[g];
    out5[3] = static_cast<uint32_t>(w->g_features[g].size());
    out5[4] = 8 * w->bin_bytes;
}
const uint32_t *synth_group_features(const void *h, uint32_t g) { return static_cast<const Workload *>(h)->g_features[g].data(); }
const uint8_t *synth_group_data(const void *h, uint32_t g) { return static_cast<const Workload *>(h)->g_data[g].data(); }
const float *synth_label(const void *h) { return static_cast<const Workload *>(h)->label.data(); }
// Query boundaries (num_queries + 1 of them) for the ranking configuration; 0 queries otherwise.
uint32_t synth_num_queries(const void *h) {
    const Workload *w = static_cast<const Workload *>(h);
    return w->query_boundaries.empty() ? 0u : static_cast<uint32_t>(w->query_boundaries.size() - 1);
}
const uint32_t *synth_query_boundaries(const void *h) { return static_cast<const Workload *>(h)->query_boundaries.data(); }
// The upper bounds of feature j (count = num_bins - nan_bin).
const double *synth_bounds(const void *h, uint32_t j) { return static_cast<const Workload *>(h)->bounds[j].data(); }

}  // extern "C"
