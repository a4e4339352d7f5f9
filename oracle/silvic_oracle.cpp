// silvic_oracle.cpp - the oracle: a CPU restatement of silvic's quantized training path.
//
// TEST INFRASTRUCTURE ONLY (see silvic_oracle.h): the checker of the HIP backend and the CPU baseline.
// Built with -ffp-contract=off and without fast math so every f64/f32 operation is the IEEE operation the
// Rust reference performs, in the same order.

#include "silvic_oracle.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <limits>
#include <memory>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------------------------------------
// Rust numeric semantics
// ---------------------------------------------------------------------------------------------------------

// `x as i64` for f64: truncation toward zero, saturating, NaN -> 0.
inline int64_t sat_i64(double x) {
    if (std::isnan(x)) return 0;
    if (x >= 9223372036854775807.0) return std::numeric_limits<int64_t>::max();
    if (x <= -9223372036854775808.0) return std::numeric_limits<int64_t>::min();
    return static_cast<int64_t>(x);
}

// `x as i32` for f32: truncation toward zero, saturating, NaN -> 0.
inline int32_t sat_i32(float x) {
    if (std::isnan(x)) return 0;
    if (x >= 2147483648.0f) return std::numeric_limits<int32_t>::max();
    if (x <= -2147483648.0f) return std::numeric_limits<int32_t>::min();
    return static_cast<int32_t>(x);
}

// f64::max: IEEE maxNum (a NaN operand yields the other).
inline double fmax_num(double a, double b) { return std::fmax(a, b); }

// f64::total_cmp as a three-way comparison.
inline int total_cmp(double a, double b) {
    int64_t x, y;
    std::memcpy(&x, &a, 8);
    std::memcpy(&y, &b, 8);
    x ^= static_cast<int64_t>(static_cast<uint64_t>(x >> 63) >> 1);
    y ^= static_cast<int64_t>(static_cast<uint64_t>(y >> 63) >> 1);
    return (x > y) - (x < y);
}

// ---------------------------------------------------------------------------------------------------------
// A small pool: parallel_for over task indices, the caller taking part.
// ---------------------------------------------------------------------------------------------------------

class Pool {
public:
    explicit Pool(int threads) { resize(threads); }
    ~Pool() { stop_workers(); }

    void resize(int threads) {
        stop_workers();
        if (threads <= 0) threads = std::max(1u, std::thread::hardware_concurrency());
        size_ = threads;
        stop_ = false;
        for (int i = 1; i < threads; ++i) workers_.emplace_back([this] { worker(); });
    }
    int size() const { return size_; }

    void run(int64_t tasks, const std::function<void(int64_t)> &fn) {
        if (tasks <= 0) return;
        if (size_ == 1 || tasks == 1) {
            for (int64_t t = 0; t < tasks; ++t) fn(t);
            return;
        }
        {
            std::unique_lock<std::mutex> lock(m_);
            job_ = &fn;
            tasks_ = tasks;
            next_.store(0);
            active_ = static_cast<int>(workers_.size());
            ++generation_;
        }
        cv_.notify_all();
        drain();
        std::unique_lock<std::mutex> lock(m_);
        done_cv_.wait(lock, [this] { return active_ == 0; });
        job_ = nullptr;
    }

private:
    void drain() {
        for (;;) {
            int64_t t = next_.fetch_add(1);
            if (t >= tasks_) break;
            (*job_)(t);
        }
    }
    void worker() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lock(m_);
                cv_.wait(lock, [&] { return stop_ || generation_ != seen; });
                if (stop_) return;
                seen = generation_;
            }
            drain();
            {
                std::unique_lock<std::mutex> lock(m_);
                if (--active_ == 0) done_cv_.notify_all();
            }
        }
    }
    void stop_workers() {
        {
            std::unique_lock<std::mutex> lock(m_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &w : workers_) w.join();
        workers_.clear();
    }

    int size_ = 1;
    std::vector<std::thread> workers_;
    std::mutex m_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(int64_t)> *job_ = nullptr;
    int64_t tasks_ = 0;
    std::atomic<int64_t> next_{0};
    int active_ = 0;
    uint64_t generation_ = 0;
    bool stop_ = false;
};

Pool &pool() {
    static Pool p(0);
    return p;
}

// parallel over [0, n) in chunks of `chunk`
void par_chunks(uint64_t n, uint64_t chunk, const std::function<void(uint64_t, uint64_t, uint64_t)> &fn) {
    uint64_t tasks = (n + chunk - 1) / chunk;
    pool().run(static_cast<int64_t>(tasks), [&](int64_t t) {
        uint64_t b = static_cast<uint64_t>(t) * chunk;
        fn(static_cast<uint64_t>(t), b, std::min(n, b + chunk));
    });
}

// ---------------------------------------------------------------------------------------------------------
// quantize.rs
// ---------------------------------------------------------------------------------------------------------

constexpr uint32_t STREAM_GRADIENT = 0;   // quantize.rs:10
constexpr uint32_t STREAM_HESSIAN = 1;    // quantize.rs:11
constexpr uint32_t STREAM_BAGGING = 2;    // quantize.rs:12
constexpr uint32_t STREAM_FEATURE_FRACTION = 3;  // split.rs:41

// quantize.rs:16-23 (lowbias32)
inline uint32_t mix32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

// quantize.rs:27-31
inline float uniform(uint32_t seed, uint32_t stream, uint32_t iteration, uint64_t row) {
    uint32_t row_hash = mix32(static_cast<uint32_t>(row) ^ mix32(static_cast<uint32_t>(row >> 32)));
    uint32_t h = mix32(seed ^ mix32(stream ^ mix32(iteration ^ row_hash)));
    return static_cast<float>(h >> 8) * (1.0f / 16777216.0f);
}

// quantize.rs:92-98
inline double positive_or_one(double v) { return (v > 0.0 && std::isfinite(v)) ? v : 1.0; }

// quantize.rs:56-84
srocm_quant_spec quant_spec(double max_abs_grad, double max_hess, std::optional<double> constant_hessian,
                            uint32_t num_bins, bool stochastic, uint32_t seed, uint32_t iteration) {
    srocm_quant_spec s{};
    s.grad_max_q = static_cast<int32_t>(num_bins / 2);
    s.hess_max_q = static_cast<int32_t>(num_bins);
    s.grad_scale = positive_or_one(max_abs_grad / static_cast<double>(s.grad_max_q));
    s.hess_scale = constant_hessian ? positive_or_one(*constant_hessian)
                                    : positive_or_one(max_hess / static_cast<double>(s.hess_max_q));
    s.inv_grad_scale = static_cast<float>(1.0 / s.grad_scale);
    s.inv_hess_scale = static_cast<float>(1.0 / s.hess_scale);
    s.constant_hessian = constant_hessian.has_value();
    s.stochastic = stochastic;
    s.seed = seed;
    s.iteration = iteration;
    return s;
}

// quantize.rs:109-122
inline int32_t quantize_grad(const srocm_quant_spec &s, float grad, uint64_t row) {
    float q;
    if (s.stochastic) {
        float u = uniform(s.seed, STREAM_GRADIENT, s.iteration, row);
        q = grad >= 0.0f ? std::trunc(std::fmaf(grad, s.inv_grad_scale, u))
                         : std::trunc(std::fmaf(grad, s.inv_grad_scale, -u));
    } else {
        q = std::nearbyint(grad * s.inv_grad_scale);
    }
    return std::clamp(sat_i32(q), -s.grad_max_q, s.grad_max_q);
}

// quantize.rs:124-136
inline int32_t quantize_hess(const srocm_quant_spec &s, float hess, uint64_t row) {
    if (s.constant_hessian) return 1;
    float q;
    if (s.stochastic) {
        float u = uniform(s.seed, STREAM_HESSIAN, s.iteration, row);
        q = std::trunc(std::fmaf(hess, s.inv_hess_scale, u));
    } else {
        q = std::nearbyint(hess * s.inv_hess_scale);
    }
    return std::clamp(sat_i32(q), 0, s.hess_max_q);
}

// quantize.rs:103-107
inline int32_t quantize_row(const srocm_quant_spec &s, float grad, float hess, uint64_t row) {
    int32_t g = quantize_grad(s, grad, row);
    int32_t h = quantize_hess(s, hess, row);
    return static_cast<int32_t>(static_cast<uint32_t>(h) * 65536u + static_cast<uint32_t>(g));
}

// quantize.rs:140-143
inline void unpack(int32_t packed, int32_t &g, int32_t &h) {
    g = static_cast<int16_t>(static_cast<uint16_t>(static_cast<uint32_t>(packed)));
    h = (packed - g) >> 16;
}

// quantize.rs:147-149
inline bool in_bag(uint32_t seed, uint32_t round, uint64_t row, double fraction) {
    return static_cast<double>(uniform(seed, STREAM_BAGGING, round, row)) < fraction;
}

// quantize.rs:153-159
float fixed_point_scale(double max_abs) {
    if (!std::isfinite(max_abs) || max_abs <= 0.0) return 1.0f;
    int32_t exponent = 30 - static_cast<int32_t>(sat_i64(std::ceil(std::log2(max_abs))));
    exponent = std::clamp(exponent, -126, 127);
    return std::ldexp(1.0f, exponent);
}

// quantize.rs:163-165
inline int64_t to_fixed(float value, float scale) { return sat_i64(static_cast<double>(std::nearbyint(value * scale))); }

// ---------------------------------------------------------------------------------------------------------
// objective/{binary,regression}.rs
// ---------------------------------------------------------------------------------------------------------

constexpr double K_EPSILON = static_cast<double>(1e-15f);  // objective/mod.rs:20, split.rs:37
constexpr uint64_t GRAD_CHUNK = 1 << 14;                     // regression.rs:56

void gradients(uint32_t objective, double sigmoid, const float *scores, const float *label, const float *weight,
               uint64_t n, float *grad, float *hess) {
    par_chunks(n, GRAD_CHUNK, [&](uint64_t, uint64_t b, uint64_t e) {
        for (uint64_t row = b; row < e; ++row) {
            if (objective == SROCM_OBJ_BINARY) {
                // binary.rs:41-47
                double sign = label[row] > 0.0f ? 1.0 : -1.0;
                double response = -sign * sigmoid / (1.0 + std::exp(sign * sigmoid * static_cast<double>(scores[row])));
                double abs_response = std::fabs(response);
                double w = weight ? static_cast<double>(weight[row]) : 1.0;
                grad[row] = static_cast<float>(response * w);
                hess[row] = static_cast<float>(abs_response * (sigmoid - abs_response) * w);
            } else {
                // regression.rs:80-90: f32 arithmetic
                float residual = scores[row] - label[row];
                if (weight) {
                    grad[row] = residual * weight[row];
                    hess[row] = weight[row];
                } else {
                    grad[row] = residual;
                    hess[row] = 1.0f;
                }
            }
        }
    });
}

// cpu.rs:774: max of |v| as f64 with f64::max
double max_abs(const float *v, uint64_t n) {
    std::vector<double> part((n + GRAD_CHUNK - 1) / GRAD_CHUNK + 1, 0.0);
    par_chunks(n, GRAD_CHUNK, [&](uint64_t t, uint64_t b, uint64_t e) {
        double m = 0.0;
        for (uint64_t i = b; i < e; ++i) m = fmax_num(m, static_cast<double>(std::fabs(v[i])));
        part[t] = m;
    });
    double m = 0.0;
    for (double p : part) m = fmax_num(m, p);
    return m;
}

// ---------------------------------------------------------------------------------------------------------
// objective/lambdarank.rs: LambdarankNDCG with f64 accumulation, and objective/mod.rs:34-62 lambdarank_setup
// ---------------------------------------------------------------------------------------------------------

constexpr size_t RANK_MAX_POSITION = 10000;        // lambdarank.rs:22
constexpr double RANK_MIN_SIGMOID_INPUT = -50.0;   // lambdarank.rs:25
constexpr size_t RANK_SIGMOID_BINS = 1024 * 1024;  // lambdarank.rs:28
constexpr double RANK_SCORE_DISTANCE_EPSILON = static_cast<double>(0.01f);  // lambdarank.rs:31
constexpr size_t RANK_QUERIES_PER_TASK = 16;       // lambdarank.rs:249

// lambdarank.rs:34-43
const std::vector<double> &rank_discounts() {
    static const std::vector<double> d = [] {
        std::vector<double> v(RANK_MAX_POSITION);
        for (size_t i = 0; i < RANK_MAX_POSITION; ++i) v[i] = 1.0 / std::log2(2.0 + static_cast<double>(i));
        return v;
    }();
    return d;
}
double rank_discount(size_t rank) {
    const auto &d = rank_discounts();
    return rank < d.size() ? d[rank] : 1.0 / std::log2(2.0 + static_cast<double>(rank));
}

// lambdarank.rs:46-116 SigmoidTable
struct SigmoidTable {
    double sigmoid, min_input, max_input, idx_factor;
    std::vector<double> values;
    explicit SigmoidTable(double s) : sigmoid(s) {
        min_input = RANK_MIN_SIGMOID_INPUT / s / 2.0;
        max_input = -min_input;
        idx_factor = static_cast<double>(RANK_SIGMOID_BINS) / (max_input - min_input);
        values.resize(RANK_SIGMOID_BINS);
        for (size_t i = 0; i < RANK_SIGMOID_BINS; ++i) {
            double score = static_cast<double>(i) / idx_factor + min_input;
            values[i] = 1.0 / (1.0 + std::exp(score * s));
        }
    }
    double get(double delta) const {
        if (delta <= min_input) return values[0];
        if (delta >= max_input) return values[RANK_SIGMOID_BINS - 1];
        // Rust's `as usize` saturates: NaN and negatives give 0, anything at or past the last bin the last
        const double x = (delta - min_input) * idx_factor;
        const double last = static_cast<double>(RANK_SIGMOID_BINS - 1);
        return values[x >= last ? RANK_SIGMOID_BINS - 1 : (x > 0.0 ? static_cast<size_t>(x) : 0)];
    }
};

const SigmoidTable &sigmoid_table(double s) {
    static std::mutex mu;
    static std::unique_ptr<SigmoidTable> last;
    std::lock_guard<std::mutex> lock(mu);
    if (!last || last->sigmoid != s) last = std::make_unique<SigmoidTable>(s);
    return *last;
}

// Rust's `as` casts of an f32 label (lambdarank.rs:172-188, :349): NaN gives 0, out-of-range values the nearest end
// of the target type, the rest truncate toward zero
int32_t as_i32(float l) {
    if (std::isnan(l)) return 0;
    if (l <= -2147483648.0f) return std::numeric_limits<int32_t>::min();
    if (l >= 2147483648.0f) return std::numeric_limits<int32_t>::max();
    return static_cast<int32_t>(l);
}
size_t as_usize(float l) {
    if (std::isnan(l) || l <= 0.0f) return 0;
    if (l >= 18446744073709551616.0f) return std::numeric_limits<size_t>::max();
    return static_cast<size_t>(l);
}

// lambdarank.rs:172-188 check_labels: 0 when every label passes, else the first failing check (1: not an integer,
// 2: negative, 3: not below the number of label gains)
int check_labels(const float *label, uint64_t n, size_t num_gains) {
    for (uint64_t r = 0; r < n; ++r) {
        const float l = label[r];
        if (std::fabs(static_cast<double>(l) - static_cast<double>(as_i32(l))) > K_EPSILON) return 1;
        if (l < 0.0f) return 2;
        if (as_usize(l) >= num_gains) return 3;
    }
    return 0;
}

// lambdarank.rs:119-139 max_dcg_at_k
double max_dcg_at_k(size_t k, const float *labels, size_t n, const std::vector<double> &label_gain) {
    std::vector<size_t> label_count(label_gain.size(), 0);
    for (size_t i = 0; i < n; ++i) label_count[as_usize(labels[i])] += 1;
    size_t top_label = label_gain.size() - 1;
    double dcg = 0.0;
    for (size_t j = 0; j < std::min(k, n); ++j) {
        while (top_label > 0 && label_count[top_label] == 0) --top_label;
        dcg += rank_discount(j) * label_gain[top_label];
        label_count[top_label] -= 1;  // wrapping_sub: label 0 may go "below zero" unchecked
    }
    return dcg;
}

// lambdarank.rs:165-170 descending_key
uint32_t descending_key(float score) {
    float z = score + 0.0f;
    uint32_t bits;
    std::memcpy(&bits, &z, 4);
    uint32_t ascending = (bits >> 31) == 1 ? ~bits : (bits | (1u << 31));
    return ~ascending;
}

struct RankSetup {
    double sigmoid = 1.0;
    bool norm = true;
    uint32_t truncation_level = 30;
    std::vector<double> label_gain, inverse_max_dcg;
};

// lambdarank.rs:254-301 query_gradients with load_ranked (:304-322), worst_score (:325-332), accumulate_pairs
// (:336-378)
void rank_query(const RankSetup &st, size_t query, const float *scores, const float *label, const float *weight,
                size_t n, float *grad, float *hess) {
    if (n == 0) return;
    const SigmoidTable &table = sigmoid_table(st.sigmoid);
    std::vector<uint64_t> keys(n);
    for (size_t row = 0; row < n; ++row) keys[row] = (static_cast<uint64_t>(descending_key(scores[row])) << 32) | row;
    std::sort(keys.begin(), keys.end());
    std::vector<size_t> order(n);
    for (size_t k = 0; k < n; ++k) order[k] = static_cast<size_t>(keys[k] & 0xffffffffull);
    std::vector<double> score(n), gain(n), discount(n), lambda(n, 0.0), hessian(n, 0.0);
    std::vector<float> lab(n);
    for (size_t k = 0; k < n; ++k) {
        score[k] = static_cast<double>(scores[order[k]]);
        lab[k] = label[order[k]];
        gain[k] = st.label_gain[as_usize(lab[k])];
        discount[k] = rank_discount(k);
    }
    size_t worst = n - 1;
    if (worst > 0 && score[worst] == -std::numeric_limits<double>::infinity()) worst -= 1;
    const bool norm_by_distance = st.norm && score[0] != score[worst];
    const double inverse_max_dcg = st.inverse_max_dcg[query];
    size_t valid = n;
    for (size_t k = 0; k < n; ++k)
        if (score[k] == -std::numeric_limits<double>::infinity()) {
            valid = k;
            break;
        }
    const double sigmoid_squared = st.sigmoid * st.sigmoid;
    double sum_lambdas = 0.0;
    const size_t last_i = std::min<size_t>(st.truncation_level, valid == 0 ? 0 : valid - 1);
    for (size_t i = 0; i < last_i; ++i) {
        double score_i = score[i], gain_i = gain[i], discount_i = discount[i];
        float label_i = lab[i];
        double lambda_i = lambda[i], hessian_i = hessian[i];
        for (size_t j = i + 1; j < valid; ++j) {
            if (lab[j] == label_i) continue;
            double sign = label_i > lab[j] ? 1.0 : -1.0;
            double delta_score = sign * (score_i - score[j]);
            double dcg_gap = sign * (gain_i - gain[j]);
            double paired_discount = std::fabs(discount_i - discount[j]);
            double delta_pair_ndcg = dcg_gap * paired_discount * inverse_max_dcg;
            if (norm_by_distance) delta_pair_ndcg /= RANK_SCORE_DISTANCE_EPSILON + std::fabs(delta_score);
            double p = table.get(delta_score);
            double p_lambda = p * (-st.sigmoid * delta_pair_ndcg);
            double p_hessian = p * (1.0 - p) * (sigmoid_squared * delta_pair_ndcg);
            lambda_i += sign * p_lambda;
            lambda[j] -= sign * p_lambda;
            hessian_i += p_hessian;
            hessian[j] += p_hessian;
            sum_lambdas -= 2.0 * p_lambda;
        }
        lambda[i] = lambda_i;
        hessian[i] = hessian_i;
    }
    double norm_factor = st.norm && sum_lambdas > 0.0 ? std::log2(1.0 + sum_lambdas) / sum_lambdas : 1.0;
    for (size_t k = 0; k < n; ++k) {
        size_t row = order[k];
        float g = static_cast<float>(lambda[k] * norm_factor);
        float h = static_cast<float>(hessian[k] * norm_factor);
        if (weight) {
            g *= weight[row];
            h *= weight[row];
        }
        grad[row] = g;
        hess[row] = h;
    }
}

// objective/mod.rs:34-62 lambdarank_setup, with lambdarank.rs:172-188 check_labels
RankSetup lambdarank_setup(const srocm_dataset *d, double sigmoid, bool norm, uint32_t truncation,
                           const double *label_gain, uint32_t num_label_gain) {
    if (!d->query_boundaries || d->num_queries == 0) throw std::runtime_error("ranking tasks require query information");
    RankSetup st;
    st.sigmoid = sigmoid;
    st.norm = norm;
    st.truncation_level = truncation;
    if (label_gain && num_label_gain) st.label_gain.assign(label_gain, label_gain + num_label_gain);
    else
        for (uint32_t i = 0; i < 31; ++i) st.label_gain.push_back(static_cast<double>((1u << i) - 1));  // config.rs:118-121
    if (check_labels(d->label, d->num_rows, st.label_gain.size())) throw std::runtime_error("bad ranking label");
    for (uint32_t q = 0; q < d->num_queries; ++q) {
        uint32_t b = d->query_boundaries[q], e = d->query_boundaries[q + 1];
        double max_dcg = max_dcg_at_k(truncation, d->label + b, e - b, st.label_gain);
        st.inverse_max_dcg.push_back(max_dcg > 0.0 ? 1.0 / max_dcg : 0.0);
    }
    return st;
}

// lambdarank.rs:190-246 gradients: every query, parallel over queries
void rank_gradients(const RankSetup &st, const srocm_dataset *d, const float *scores, float *grad, float *hess) {
    par_chunks(d->num_queries, RANK_QUERIES_PER_TASK, [&](uint64_t, uint64_t qb, uint64_t qe) {
        for (uint64_t q = qb; q < qe; ++q) {
            uint32_t b = d->query_boundaries[q], e = d->query_boundaries[q + 1];
            rank_query(st, q, scores + b, d->label + b, d->weight ? d->weight + b : nullptr, e - b, grad + b, hess + b);
        }
    });
}

// objective/mod.rs:92-109, binary.rs:11-25, regression.rs:60-67
double init_score(uint32_t objective, double sigmoid, const float *label, const float *weight, uint64_t n) {
    double sum_label = 0.0, sum_weight = 0.0;
    if (objective == SROCM_OBJ_BINARY) {
        if (weight) {
            for (uint64_t i = 0; i < n; ++i) {
                float pos = label[i] > 0.0f ? 1.0f : 0.0f;
                sum_label = sum_label + static_cast<double>(pos * weight[i]);
                sum_weight = sum_weight + static_cast<double>(weight[i]);
            }
        } else {
            for (uint64_t i = 0; i < n; ++i) sum_label += label[i] > 0.0f ? 1.0 : 0.0;
            sum_weight = static_cast<double>(n);
        }
        double p = std::clamp(sum_label / sum_weight, K_EPSILON, 1.0 - K_EPSILON);
        double score = std::log(p / (1.0 - p)) / sigmoid;
        return std::fabs(score) > K_EPSILON ? score : 0.0;
    }
    if (weight) {
        for (uint64_t i = 0; i < n; ++i) {
            sum_label = sum_label + static_cast<double>(label[i] * weight[i]);
            sum_weight = sum_weight + static_cast<double>(weight[i]);
        }
    } else {
        for (uint64_t i = 0; i < n; ++i) sum_label += static_cast<double>(label[i]);
        sum_weight = static_cast<double>(n);
    }
    double score = sum_label / sum_weight;
    return std::fabs(score) > K_EPSILON ? score : 0.0;
}

// ---------------------------------------------------------------------------------------------------------
// backend/cpu.rs: histograms, partition, leaf sums, add_tree
// ---------------------------------------------------------------------------------------------------------

constexpr size_t MIN_ADDS_PER_BIN = 16;      // cpu.rs:26
constexpr size_t MAX_BLOCKS_PER_GROUP = 64;  // cpu.rs:29
constexpr size_t SCRATCH_BINS = 256;         // cpu.rs:31
constexpr size_t DENSE_RUN_NUM = 3;          // cpu.rs:39
constexpr size_t DENSE_RUN_DEN = 4;          // cpu.rs:40
constexpr uint64_t ROW_CHUNK = 8192;         // cpu.rs:42

// A group's bits per bin: 8 (0 means 8, silvic's bytes), or the extensions 16 and 4.
inline uint32_t group_bits(const srocm_group &g) { return g.bin_bits == 0 ? 8u : g.bin_bits; }

// cpu.rs:46-99 GroupLayout
struct GroupLayout {
    size_t group = 0, stride = 0, hist_offset = 0, bins = 0;
    size_t bits = 8;  // 16: u16 bins, 4: two bins a byte (extensions; no counterpart in cpu.rs)
    std::vector<int64_t> column_features;  // -1: no feature
    std::vector<size_t> offsets;
    std::vector<std::pair<uint32_t, uint32_t>> runs;
    size_t adds = 0;

    void activate(const uint8_t *used, size_t num_features) {
        runs.clear();
        auto wanted = [&](int64_t f) {
            if (!used) return true;
            return static_cast<size_t>(f) < num_features ? used[f] != 0 : true;
        };
        size_t width = column_features.size();
        size_t active = 0;
        for (int64_t f : column_features)
            if (f >= 0 && wanted(f)) ++active;
        if (active == 0) {
            adds = 0;
            return;
        }
        if (active * DENSE_RUN_DEN >= width * DENSE_RUN_NUM) {
            runs.emplace_back(0, static_cast<uint32_t>(width));
            adds = width;
            return;
        }
        adds = active;
        std::optional<size_t> start;
        for (size_t column = 0; column < width; ++column) {
            bool on = column_features[column] >= 0 && wanted(column_features[column]);
            if (on && !start) start = column;
            else if (!on && start) {
                runs.emplace_back(static_cast<uint32_t>(*start), static_cast<uint32_t>(column));
                start.reset();
            }
        }
        if (start) runs.emplace_back(static_cast<uint32_t>(*start), static_cast<uint32_t>(width));
    }
};

// cpu.rs:178-223
std::vector<GroupLayout> group_layout(const srocm_dataset *d) {
    std::vector<GroupLayout> out;
    for (uint32_t gi = 0; gi < d->num_groups; ++gi) {
        const srocm_group &g = d->groups[gi];
        GroupLayout L;
        L.group = gi;
        L.bins = g.total_bins;
        L.stride = g.row_stride;
        L.hist_offset = g.hist_offset;
        L.bits = group_bits(g);
        if (L.bits != 4 && L.bits != 8 && L.bits != 16) throw std::runtime_error("a group's bins are 4, 8 or 16 bits");
        size_t width = 0;
        for (uint32_t k = 0; k < g.num_features; ++k)
            width = std::max<size_t>(width, d->features[g.features[k]].column + 1);
        L.column_features.assign(width, -1);
        L.offsets.assign(width, L.bins);
        for (uint32_t k = 0; k < g.num_features; ++k) {
            uint32_t f = g.features[k];
            const srocm_feature &m = d->features[f];
            const size_t end_byte = L.bits == 4 ? m.column / 2 + 1 : m.column + L.bits / 8;
            if (m.hist_offset < g.hist_offset || m.hist_offset - g.hist_offset + m.num_bins > L.bins || end_byte > L.stride)
                throw std::runtime_error("feature lies outside its group's bins or row");
            if (L.bits == 16 && (m.kind != SROCM_BINS_NUMERICAL || m.num_bins > 1024))
                throw std::runtime_error("a 2-byte group holds numerical features of at most 1024 bins");
            if (L.bits == 8 && m.num_bins > 256) throw std::runtime_error("a feature of more than 256 byte bins");
            if (L.bits == 4 && m.num_bins > 16) throw std::runtime_error("a feature of more than 16 4-bit bins");
            L.column_features[m.column] = f;
            L.offsets[m.column] = m.hist_offset - g.hist_offset;
        }
        L.activate(nullptr, d->num_features);
        out.push_back(std::move(L));
    }
    return out;
}

// cpu.rs:347-351
size_t block_rows(size_t rows, const GroupLayout &g) {
    size_t adds_per_row = std::max<size_t>(g.adds, 1);
    size_t min_rows = (MIN_ADDS_PER_BIN * g.bins + adds_per_row - 1) / adds_per_row;
    return std::max<size_t>(std::max(min_rows, (rows + MAX_BLOCKS_PER_GROUP - 1) / MAX_BLOCKS_PER_GROUP), 1);
}

// The u16 bin at byte offset `column` of a row (2-byte groups).
inline uint32_t bin16(const uint8_t *row, size_t column) {
    return static_cast<uint32_t>(row[column]) | (static_cast<uint32_t>(row[column + 1]) << 8);
}

// The 4-bit bin in slot `column` of a row (two to a byte, the low half first).
inline uint32_t bin4(const uint8_t *row, size_t column) { return (row[column / 2] >> (4 * (column % 2))) & 15u; }

// The bin of a row's feature in column `column` of a group (a byte offset, or a 4-bit slot).
inline uint32_t bin_at(const srocm_group &g, size_t row, size_t column) {
    const uint8_t *r = g.data + row * g.row_stride;
    const uint32_t bits = group_bits(g);
    return bits == 16 ? bin16(r, column) : (bits == 4 ? bin4(r, column) : r[column]);
}

// cpu.rs:307-314 add_run, cpu.rs:277-304 accumulate_rows (prefetching left to the hardware). A 16-bit group adds
// its features' u16 bins, a 4-bit group its features' half-byte bins; every add is an exact integer one, so the
// order of the adds changes nothing.
inline void accumulate(const GroupLayout &g, const uint8_t *data, const uint32_t *rows, const int64_t *values,
                       size_t n, int64_t *acc) {
    if (g.bits != 8) {
        for (size_t i = 0; i < n; ++i) {
            const uint8_t *row = data + static_cast<size_t>(rows[i]) * g.stride;
            int64_t v = values[i];
            for (const auto &run : g.runs)
                for (uint32_t c = run.first; c < run.second; ++c)
                    if (g.column_features[c] >= 0) acc[g.offsets[c] + (g.bits == 16 ? bin16(row, c) : bin4(row, c))] += v;
        }
        return;
    }
    size_t width = g.runs.empty() ? 0 : g.runs.back().second;
    for (size_t i = 0; i < n; ++i) {
        const uint8_t *bins = data + static_cast<size_t>(rows[i]) * g.stride;
        int64_t v = values[i];
        for (const auto &run : g.runs)
            for (uint32_t c = run.first; c < run.second; ++c) acc[g.offsets[c] + bins[c]] += v;
        (void)width;
    }
}

// cpu.rs:517-525 flush_packed
inline void flush_packed(int64_t *acc, double *sums, size_t len) {
    for (size_t i = 0; i < len; ++i) {
        int64_t value = acc[i];
        int64_t g = static_cast<int32_t>(value);
        sums[2 * i] += static_cast<double>(g);
        sums[2 * i + 1] += static_cast<double>((value - g) >> 32);
        acc[i] = 0;
    }
}

struct BlockTask {
    size_t group, start, end;
};

// cpu.rs:479-513 histogram_quantized (with histogram_blocks cpu.rs:374-415 and merge_blocks cpu.rs:419-463)
void histogram_quantized(const srocm_dataset *d, const std::vector<GroupLayout> &layout, const int32_t *packed,
                         int64_t max_quant, const uint32_t *rows, size_t n, double *out) {
    size_t row_limit = static_cast<size_t>(static_cast<int64_t>(INT32_MAX) / std::max<int64_t>(max_quant, 1));
    // ordered gradients (cpu.rs:466-476)
    std::vector<int64_t> gh(n);
    par_chunks(n, ROW_CHUNK, [&](uint64_t, uint64_t b, uint64_t e) {
        for (uint64_t i = b; i < e; ++i) {
            int32_t g, h;
            unpack(packed[rows[i]], g, h);
            gh[i] = (static_cast<int64_t>(h) << 32) + static_cast<int64_t>(g);
        }
    });
    std::vector<BlockTask> tasks;
    for (size_t gi = 0; gi < layout.size(); ++gi) {
        if (layout[gi].adds == 0) continue;
        size_t size = block_rows(n, layout[gi]);
        size_t count = std::max<size_t>((n + size - 1) / size, 1);
        for (size_t b = 0; b < count; ++b) tasks.push_back({gi, std::min(b * size, n), std::min((b + 1) * size, n)});
    }
    std::vector<size_t> slot_offset(tasks.size() + 1, 0);
    for (size_t t = 0; t < tasks.size(); ++t)
        slot_offset[t + 1] = slot_offset[t] + 2 * (layout[tasks[t].group].bins + SCRATCH_BINS);
    std::vector<double> sums(slot_offset.back(), 0.0);
    pool().run(static_cast<int64_t>(tasks.size()), [&](int64_t t) {
        const BlockTask &task = tasks[t];
        const GroupLayout &g = layout[task.group];
        const uint8_t *data = d->groups[g.group].data;
        double *s = sums.data() + slot_offset[t];
        std::vector<int64_t> acc(g.bins + SCRATCH_BINS, 0);
        for (size_t b = task.start; b < task.end; b += row_limit) {
            size_t e = std::min(task.end, b + row_limit);
            accumulate(g, data, rows + b, gh.data() + b, e - b, acc.data());
            flush_packed(acc.data(), s, acc.size());
        }
    });
    // merge in block order; bins outside every group, and of groups without blocks, are zero
    std::fill(out, out + 2 * d->total_bins, 0.0);
    for (size_t gi = 0; gi < layout.size(); ++gi) {
        const GroupLayout &g = layout[gi];
        double *target = out + 2 * g.hist_offset;
        bool first = true;
        for (size_t t = 0; t < tasks.size(); ++t) {
            if (tasks[t].group != gi) continue;
            const double *s = sums.data() + slot_offset[t];
            if (first) {
                std::copy(s, s + 2 * g.bins, target);
                first = false;
            } else {
                for (size_t i = 0; i < 2 * g.bins; ++i) target[i] += s[i];
            }
        }
    }
}

// cpu.rs:556-599 stable_partition, by chunks of ROW_CHUNK through a scratch buffer
uint32_t stable_partition(uint32_t *rows, size_t n, const std::function<bool(uint32_t)> &goes_left) {
    std::vector<uint32_t> scratch(n);
    size_t chunks = (n + ROW_CHUNK - 1) / ROW_CHUNK;
    std::vector<size_t> lefts(chunks, 0);
    par_chunks(n, ROW_CHUNK, [&](uint64_t c, uint64_t b, uint64_t e) {
        size_t left = b, right = e;
        for (uint64_t i = b; i < e; ++i) {
            uint32_t row = rows[i];
            if (goes_left(row)) scratch[left++] = row;
            else scratch[--right] = row;
        }
        std::reverse(scratch.begin() + static_cast<long>(left), scratch.begin() + static_cast<long>(e));
        lefts[c] = left - b;
    });
    size_t total_left = 0;
    for (size_t l : lefts) total_left += l;
    std::vector<size_t> lpos(chunks), rpos(chunks);
    size_t lp = 0, rp = total_left;
    for (size_t c = 0; c < chunks; ++c) {
        size_t len = std::min<size_t>(ROW_CHUNK, n - c * ROW_CHUNK);
        lpos[c] = lp;
        rpos[c] = rp;
        lp += lefts[c];
        rp += len - lefts[c];
    }
    par_chunks(n, ROW_CHUNK, [&](uint64_t c, uint64_t b, uint64_t e) {
        size_t l = lefts[c];
        std::copy(scratch.begin() + static_cast<long>(b), scratch.begin() + static_cast<long>(b + l), rows + lpos[c]);
        std::copy(scratch.begin() + static_cast<long>(b + l), scratch.begin() + static_cast<long>(e), rows + rpos[c]);
    });
    return static_cast<uint32_t>(total_left);
}

// BinSplit::goes_left (backend/mod.rs:34-37); a split on a 2-byte group's feature carries a numerical rule in its
// words (threshold, NaN bin + 1 when missing values go left), since a mask of up to 1024 bins does not fit.
inline bool goes_left(const srocm_bin_split &s, uint32_t bin, bool wide) {
    if (wide) return bin <= s.left_bins[0] || (s.left_bins[1] != 0 && bin == s.left_bins[1] - 1);
    return (s.left_bins[bin / 32] >> (bin % 32)) & 1u;
}

// cpu.rs:666-695 add_tree_to (a plain walk: the reference's branch-free walk visits the same nodes)
void add_tree_to(const srocm_dataset *d, const srocm_device_node *nodes, uint32_t num_nodes,
                 const float *leaf_values, uint32_t num_leaves, float *scores) {
    uint64_t n = d->num_rows;
    if (num_nodes == 0) {
        float v = leaf_values[0];
        par_chunks(n, ROW_CHUNK, [&](uint64_t, uint64_t b, uint64_t e) {
            for (uint64_t i = b; i < e; ++i) scores[i] += v;
        });
        return;
    }
    for (uint32_t k = 0; k < num_nodes; ++k) {
        const srocm_device_node &nd = nodes[k];
        if (nd.split.group >= d->num_groups) throw std::runtime_error("malformed device tree");
        for (int32_t c : {nd.left, nd.right}) {
            if (c >= 0 ? (static_cast<uint32_t>(c) <= k || static_cast<uint32_t>(c) >= num_nodes)
                       : (static_cast<uint32_t>(~c) >= num_leaves))
                throw std::runtime_error("malformed device tree");
        }
    }
    par_chunks(n, ROW_CHUNK, [&](uint64_t, uint64_t b, uint64_t e) {
        for (uint64_t row = b; row < e; ++row) {
            int32_t node = 0;
            while (node >= 0) {
                const srocm_device_node &nd = nodes[node];
                const srocm_group &g = d->groups[nd.split.group];
                node = goes_left(nd.split, bin_at(g, row, nd.split.column), group_bits(g) == 16) ? nd.left : nd.right;
            }
            scores[row] += leaf_values[~node];
        }
    });
}

// ---------------------------------------------------------------------------------------------------------
// split.rs
// ---------------------------------------------------------------------------------------------------------

constexpr double MIN_SCORE = -std::numeric_limits<double>::infinity();  // split.rs:39
constexpr size_t MAX_BINS = 1024;  // split.rs:43 has 256, silvic's largest feature; 2-byte features take 1024

// split.rs:145-154
inline double sign_of(double x) { return static_cast<double>(static_cast<int>(x > 0.0) - static_cast<int>(x < 0.0)); }
inline double threshold_l1(double s, double l1) {
    double reg = fmax_num(std::fabs(s) - l1, 0.0);
    return sign_of(s) * reg;
}
// split.rs:159-162
inline double leaf_gain(double g, double h, double l1, double l2) {
    double r = fmax_num(std::fabs(g) - l1, 0.0);
    return r * r / (h + l2);
}
// split.rs:167-186 (the scalar path)
inline double split_gain(double g0, double g1, double h0, double h1, double l1, double l2) {
    return leaf_gain(g0, h0, l1, l2) + leaf_gain(g1, h1, l1, l2);
}
// split.rs:190-192
inline double leaf_output(double g, double h, double l1, double l2) { return -threshold_l1(g, l1) / (h + l2); }
// split.rs:196-198
inline int64_t round_int(double x) { return sat_i64(x + 0.5); }

struct LeafSums {
    double grad = 0.0, hess = 0.0;
    int64_t count = 0;
};

// split.rs:201-259
struct LeafCtx {
    const srocm_split_config *cfg;
    double scale_grad, scale_hess;
    LeafSums units;
    double sum_grad, sum_hess;
    int64_t num_data;
    double cnt_factor;
    double min_gain_shift;

    static std::optional<LeafCtx> make(const srocm_split_config *cfg, double sg, double sh, LeafSums units) {
        if (std::isnan(units.hess) || units.hess <= 0.0 || units.count <= 0) return std::nullopt;
        LeafCtx c;
        c.cfg = cfg;
        c.scale_grad = sg;
        c.scale_hess = sh;
        c.units = units;
        c.sum_grad = units.grad * sg;
        c.sum_hess = units.hess * sh + 2.0 * K_EPSILON;
        double gain_shift = leaf_gain(c.sum_grad, c.sum_hess, cfg->lambda_l1, cfg->lambda_l2);
        c.num_data = units.count;
        c.cnt_factor = static_cast<double>(units.count) / c.sum_hess;
        c.min_gain_shift = gain_shift + cfg->min_gain_to_split;
        return c;
    }
    int64_t bin_count(double hess_units) const { return round_int(hess_units * scale_hess * cnt_factor); }
};

enum class Check { Continue, Break, Evaluate };

// split.rs:267-296
struct Side {
    double units[2] = {0.0, 0.0};
    int64_t count = 0;
    double hess = K_EPSILON;
    void add(const LeafCtx &ctx, const double *bin) {
        units[0] += bin[0];
        units[1] += bin[1];
        count += ctx.bin_count(bin[1]);
        hess = K_EPSILON + units[1] * ctx.scale_hess;
    }
    double grad(const LeafCtx &ctx) const { return units[0] * ctx.scale_grad; }
};

// split.rs:243-258
Check check(const LeafCtx &ctx, const Side &grow, int64_t shrink_count, double shrink_hess) {
    const srocm_split_config &c = *ctx.cfg;
    if (grow.count < c.min_data_in_leaf || grow.count <= 0 || grow.hess < c.min_sum_hessian_in_leaf ||
        grow.units[1] <= 0.0)
        return Check::Continue;
    if (shrink_count < c.min_data_in_leaf || shrink_count <= 0) return Check::Break;
    if (shrink_hess < c.min_sum_hessian_in_leaf || ctx.units.hess - grow.units[1] <= 0.0) return Check::Break;
    return Check::Evaluate;
}

// split.rs:298-307
struct Best {
    double gain = 0.0;
    uint32_t threshold = 0;
    double left_grad = 0.0, left_hess = 0.0;
    int64_t left_count = 0;
    double left_units[2] = {0.0, 0.0};
};

enum class Kind { Numerical, OneHot, Sorted };

// split.rs:310-317
struct Candidate {
    size_t feature = 0;
    double gain = 0.0;
    Best best;
    Kind kind = Kind::Numerical;
    bool default_left = false;  // Numerical
    bool forward = false;       // Sorted
};

// split.rs:344-352
struct Grown {
    size_t bin = 0;
    double units[2] = {0.0, 0.0};
    int64_t count = 0;
    double gain = 0.0;
};

// split.rs:386-532 ScanBuffer: running sums, then gains, then the first maximum
struct ScanBuffer {
    uint16_t bin[MAX_BINS];
    double grad[MAX_BINS], hess[MAX_BINS];
    int64_t count[MAX_BINS];
    double gain[MAX_BINS];

    // split.rs:420-444 fill, over (t, bin) pairs given as a sequence of bin indices
    size_t fill(const LeafCtx &ctx, const double *hist, const std::vector<size_t> &order) {
        const srocm_split_config &cfg = *ctx.cfg;
        int64_t min_count = std::max<int64_t>(cfg.min_data_in_leaf, 1);
        double min_hess = cfg.min_sum_hessian_in_leaf;
        double g = 0.0, uh = 0.0;
        int64_t cnt = 0;
        size_t len = 0;
        for (size_t k = 0; k < order.size() && k < MAX_BINS; ++k) {
            size_t t = order[k];
            const double *b = hist + 2 * t;
            g += b[0];
            uh += b[1];
            cnt += round_int(b[1] * ctx.scale_hess * ctx.cnt_factor);
            double h = K_EPSILON + uh * ctx.scale_hess;
            bool skip = cnt < min_count || h < min_hess || uh <= 0.0;
            bool other_small = ctx.num_data - cnt < min_count || ctx.sum_hess - h < min_hess || ctx.units.hess - uh <= 0.0;
            if (other_small && !skip) break;
            bin[k] = static_cast<uint16_t>(t);
            grad[k] = g;
            hess[k] = uh;
            count[k] = cnt;
            len = k + 1;
        }
        return len;
    }

    // split.rs:447-462 evaluate
    void evaluate(const LeafCtx &ctx, size_t len) {
        const srocm_split_config &cfg = *ctx.cfg;
        int64_t min_count = std::max<int64_t>(cfg.min_data_in_leaf, 1);
        for (size_t k = 0; k < len; ++k) {
            double uh = hess[k];
            double h = K_EPSILON + uh * ctx.scale_hess;
            bool skip = count[k] < min_count || h < cfg.min_sum_hessian_in_leaf || uh <= 0.0;
            double gg = grad[k] * ctx.scale_grad;
            double gn = split_gain(ctx.sum_grad - gg, gg, ctx.sum_hess - h, h, cfg.lambda_l1, cfg.lambda_l2);
            gain[k] = skip ? -std::numeric_limits<double>::infinity() : gn;
        }
    }

    // split.rs:508-531 best
    std::optional<Grown> best(const LeafCtx &ctx, size_t stop) const {
        double m = -std::numeric_limits<double>::infinity();
        for (size_t k = 0; k < stop; ++k) m = fmax_num(m, gain[k]);
        if (!(m > ctx.min_gain_shift)) return std::nullopt;
        for (size_t k = 0; k < stop; ++k) {
            if (gain[k] == m) {
                Grown g;
                g.bin = bin[k];
                g.units[0] = grad[k];
                g.units[1] = hess[k];
                g.count = count[k];
                g.gain = gain[k];
                return g;
            }
        }
        return std::nullopt;
    }

    // split.rs:400-405 complete
    std::optional<Grown> complete(const LeafCtx &ctx, size_t len, bool &splittable) {
        evaluate(ctx, len);
        auto b = best(ctx, len);
        splittable |= b.has_value();
        return b;
    }
};

// split.rs:557-567
Best reverse_best(const LeafCtx &ctx, const Grown &right) {
    double right_hess = K_EPSILON + right.units[1] * ctx.scale_hess;
    Best b;
    b.gain = right.gain;
    b.threshold = static_cast<uint32_t>(right.bin - 1);
    b.left_grad = ctx.sum_grad - right.units[0] * ctx.scale_grad;
    b.left_hess = ctx.sum_hess - right_hess;
    b.left_count = ctx.num_data - right.count;
    b.left_units[0] = ctx.units.grad - right.units[0];
    b.left_units[1] = ctx.units.hess - right.units[1];
    return b;
}

// split.rs:571-580
Best forward_best(const LeafCtx &ctx, const Grown &left) {
    Best b;
    b.gain = left.gain;
    b.threshold = static_cast<uint32_t>(left.bin);
    b.left_grad = left.units[0] * ctx.scale_grad;
    b.left_hess = K_EPSILON + left.units[1] * ctx.scale_hess;
    b.left_count = left.count;
    b.left_units[0] = left.units[0];
    b.left_units[1] = left.units[1];
    return b;
}

struct FeatureResult {
    bool splittable = false;
    std::optional<Candidate> best;
};

Candidate make_candidate(const LeafCtx &ctx, size_t feature, const Best &b, Kind kind) {
    Candidate c;
    c.feature = feature;
    c.gain = b.gain - ctx.min_gain_shift;
    c.best = b;
    c.kind = kind;
    return c;
}

struct Scans {
    ScanBuffer reverse, forward;
};

// split.rs:584-620 find_numerical
FeatureResult find_numerical(const LeafCtx &ctx, Scans &scans, size_t feature, const double *hist, size_t num_bins,
                             bool nan_bin) {
    bool splittable = false;
    std::optional<std::pair<Best, bool>> result;
    if (nan_bin && num_bins > 2) {
        size_t last = num_bins - 2;
        std::vector<size_t> rev, fwd;
        for (size_t t = last; t >= 1; --t) rev.push_back(t);
        for (size_t t = 0; t <= last; ++t) fwd.push_back(t);
        size_t reverse_len = scans.reverse.fill(ctx, hist, rev);
        size_t forward_len = scans.forward.fill(ctx, hist, fwd);
        double output_gain = MIN_SCORE;
        if (auto right = scans.reverse.complete(ctx, reverse_len, splittable)) {
            Best b = reverse_best(ctx, *right);
            output_gain = b.gain - ctx.min_gain_shift;
            result = std::make_pair(b, true);
        }
        if (auto left = scans.forward.complete(ctx, forward_len, splittable)) {
            Best b = forward_best(ctx, *left);
            if (b.gain > output_gain + ctx.min_gain_shift) result = std::make_pair(b, false);
        }
    } else if (num_bins >= 2) {
        std::vector<size_t> rev;
        for (size_t t = num_bins - 1; t >= 1; --t) rev.push_back(t);
        size_t len = scans.reverse.fill(ctx, hist, rev);
        if (auto right = scans.reverse.complete(ctx, len, splittable)) result = std::make_pair(reverse_best(ctx, *right), !nan_bin);
    }
    FeatureResult r;
    r.splittable = splittable;
    if (result) {
        Candidate c = make_candidate(ctx, feature, result->first, Kind::Numerical);
        c.default_left = result->second;
        r.best = c;
    }
    return r;
}

// split.rs:695-736 find_onehot
FeatureResult find_onehot(const LeafCtx &ctx, size_t feature, const double *hist, size_t num_bins) {
    const srocm_split_config &cfg = *ctx.cfg;
    bool splittable = false;
    std::optional<Best> best;
    for (size_t t = 1; t < num_bins; ++t) {
        const double *bin = hist + 2 * t;
        Side left;
        left.add(ctx, bin);
        int64_t other_count = ctx.num_data - left.count;
        double raw_hess = bin[1] * ctx.scale_hess;
        double other_hess = ctx.sum_hess - raw_hess - K_EPSILON;
        Side grow = left;
        grow.hess = raw_hess;
        if (check(ctx, grow, other_count, other_hess) != Check::Evaluate) continue;
        double grad = left.grad(ctx);
        double gain = split_gain(ctx.sum_grad - grad, grad, other_hess, raw_hess + K_EPSILON, cfg.lambda_l1, cfg.lambda_l2);
        if (std::isnan(gain) || gain <= ctx.min_gain_shift) continue;
        splittable = true;
        if (!best || gain > best->gain) {
            Best b;
            b.gain = gain;
            b.threshold = static_cast<uint32_t>(t);
            b.left_grad = grad;
            b.left_hess = raw_hess + K_EPSILON;
            b.left_count = left.count;
            b.left_units[0] = left.units[0];
            b.left_units[1] = left.units[1];
            best = b;
        }
    }
    FeatureResult r;
    r.splittable = splittable;
    if (best) r.best = make_candidate(ctx, feature, *best, Kind::OneHot);
    return r;
}

// split.rs:740-760 sorted_categories
std::vector<uint16_t> sorted_categories(const LeafCtx &ctx, const double *hist, size_t num_bins_in) {
    const srocm_split_config &cfg = *ctx.cfg;
    size_t num_bins = std::min(num_bins_in, MAX_BINS);
    std::vector<uint16_t> order;
    for (size_t t = 1; t < num_bins; ++t)
        if (static_cast<double>(ctx.bin_count(hist[2 * t + 1])) >= cfg.cat_smooth) order.push_back(static_cast<uint16_t>(t));
    auto ctr = [&](uint16_t t) {
        return (hist[2 * t] * ctx.scale_grad) / (hist[2 * t + 1] * ctx.scale_hess + cfg.cat_smooth);
    };
    std::sort(order.begin(), order.end(), [&](uint16_t a, uint16_t b) {
        int c = total_cmp(ctr(a), ctr(b));
        if (c != 0) return c < 0;
        return a < b;
    });
    return order;
}

// split.rs:795-843 SortedScan::run
std::optional<Best> sorted_run(const LeafCtx &ctx, const double *hist, double l2, size_t steps,
                               const std::function<size_t(size_t)> &order, bool &splittable) {
    const srocm_split_config &cfg = *ctx.cfg;
    Side left;
    int64_t cnt_cur_group = 0;
    std::optional<Best> best;
    for (size_t i = 0; i < steps; ++i) {
        size_t t = order(i);
        int64_t before = left.count;
        left.add(ctx, hist + 2 * t);
        cnt_cur_group += left.count - before;
        int64_t right_count = ctx.num_data - left.count;
        double right_hess = ctx.sum_hess - left.hess;
        Check c = check(ctx, left, right_count, right_hess);
        if (c == Check::Continue) continue;
        if (c == Check::Break) break;
        if (right_count < cfg.min_data_per_group) break;
        if (cnt_cur_group < cfg.min_data_per_group) continue;
        cnt_cur_group = 0;
        double left_grad = left.grad(ctx);
        double gain = split_gain(left_grad, ctx.sum_grad - left_grad, left.hess, right_hess, cfg.lambda_l1, l2);
        if (std::isnan(gain) || gain <= ctx.min_gain_shift) continue;
        splittable = true;
        if (!best || gain > best->gain) {
            Best b;
            b.gain = gain;
            b.threshold = static_cast<uint32_t>(i);
            b.left_grad = left_grad;
            b.left_hess = left.hess;
            b.left_count = left.count;
            b.left_units[0] = left.units[0];
            b.left_units[1] = left.units[1];
            best = b;
        }
    }
    return best;
}

// split.rs:764-784 find_sorted_categorical
FeatureResult find_sorted_categorical(const LeafCtx &ctx, size_t feature, const double *hist, size_t num_bins) {
    const srocm_split_config &cfg = *ctx.cfg;
    std::vector<uint16_t> sorted = sorted_categories(ctx, hist, num_bins);
    size_t used_bin = sorted.size();
    size_t max_num_cat = std::min<size_t>(cfg.max_cat_threshold, (used_bin + 1) / 2);
    double l2 = cfg.lambda_l2 + cfg.cat_l2;
    bool splittable = false;
    std::optional<std::pair<Best, bool>> best;
    for (bool forward : {true, false}) {
        auto order = [&](size_t i) -> size_t { return forward ? sorted[i] : sorted[used_bin - 1 - i]; };
        if (auto cand = sorted_run(ctx, hist, l2, std::min(used_bin, max_num_cat), order, splittable)) {
            if (!best || cand->gain > best->first.gain) best = std::make_pair(*cand, forward);
        }
    }
    FeatureResult r;
    r.splittable = splittable;
    if (best) {
        Candidate c = make_candidate(ctx, feature, best->first, Kind::Sorted);
        c.forward = best->second;
        r.best = c;
    }
    return r;
}

// split.rs:847-862
FeatureResult find_feature(const LeafCtx &ctx, Scans &scans, size_t feature, const srocm_feature &meta,
                           const double *hist) {
    switch (meta.kind) {
    case SROCM_BINS_NUMERICAL:
        return find_numerical(ctx, scans, feature, hist, meta.num_bins, meta.nan_bin != 0);
    case SROCM_BINS_CATEGORICAL:
        if (meta.num_bins <= ctx.cfg->max_cat_to_onehot) return find_onehot(ctx, feature, hist, meta.num_bins);
        return find_sorted_categorical(ctx, feature, hist, meta.num_bins);
    default:
        return FeatureResult{};
    }
}

// split.rs:866-880
bool better(const Candidate &a, const Candidate &b) {
    auto gain = [](const Candidate &s) { return std::isnan(s.gain) ? MIN_SCORE : s.gain; };
    double ga = gain(a), gb = gain(b);
    if (ga > gb) return true;
    if (ga < gb) return false;
    return a.feature < b.feature;
}

std::optional<Candidate> best_of(std::optional<Candidate> a, std::optional<Candidate> b) {
    if (a && b) return better(*b, *a) ? b : a;
    return a ? a : b;
}

// split.rs:632-651 finish + split.rs:654-692 split_info
oracle_split_info split_info(const LeafCtx &ctx, const double *hist, const srocm_feature &meta, const Candidate &c) {
    oracle_split_info out{};
    const Best &b = c.best;
    double l1 = ctx.cfg->lambda_l1;
    double l2 = ctx.cfg->lambda_l2;
    out.found = 1;
    out.feature = static_cast<int32_t>(c.feature);
    out.gain = b.gain - ctx.min_gain_shift;
    if (c.kind == Kind::Numerical) {
        out.categorical = 0;
        out.threshold = b.threshold;
        out.default_left = c.default_left;
    } else if (c.kind == Kind::OneHot) {
        out.categorical = 1;
        out.num_cat_bins = 1;
        out.cat_bins[0] = b.threshold;
    } else {
        out.categorical = 1;
        std::vector<uint16_t> sorted = sorted_categories(ctx, hist, meta.num_bins);
        size_t take = b.threshold + 1;
        out.num_cat_bins = static_cast<uint32_t>(take);
        for (size_t i = 0; i < take; ++i) out.cat_bins[i] = c.forward ? sorted[i] : sorted[sorted.size() - 1 - i];
        l2 = ctx.cfg->lambda_l2 + ctx.cfg->cat_l2;
    }
    out.left.grad = b.left_units[0];
    out.left.hess = b.left_units[1];
    out.left.count = b.left_count;
    out.right.grad = ctx.units.grad - b.left_units[0];
    out.right.hess = ctx.units.hess - b.left_units[1];
    out.right.count = ctx.num_data - b.left_count;
    out.left_output = leaf_output(b.left_grad, b.left_hess, l1, l2);
    out.right_output = leaf_output(ctx.sum_grad - b.left_grad, ctx.sum_hess - b.left_hess, l1, l2);
    return out;
}

// split.rs:919-961 (results do not depend on how features are grouped: `better` is a total order)
oracle_split_info find_best_split(const double *hist, const srocm_feature *features, size_t nf, const uint8_t *evaluate,
                                  LeafSums sums, double gs, double hs, const srocm_split_config *cfg,
                                  uint8_t *splittable) {
    std::fill(splittable, splittable + nf, 0);
    oracle_split_info none{};
    auto ctx = LeafCtx::make(cfg, gs, hs, sums);
    if (!ctx) return none;
    constexpr size_t CHUNK = 16;
    size_t chunks = (nf + CHUNK - 1) / CHUNK;
    std::vector<std::optional<Candidate>> bests(chunks);
    pool().run(static_cast<int64_t>(chunks), [&](int64_t ch) {
        auto scans = std::make_unique<Scans>();
        std::optional<Candidate> best;
        for (size_t f = ch * CHUNK; f < std::min(nf, (ch + 1) * CHUNK); ++f) {
            const srocm_feature &m = features[f];
            if (!evaluate[f] || m.num_bins == 0 || m.kind == SROCM_BINS_TRIVIAL) continue;
            FeatureResult r = find_feature(*ctx, *scans, f, m, hist + 2 * static_cast<size_t>(m.hist_offset));
            splittable[f] = r.splittable;
            best = best_of(best, r.best);
        }
        bests[ch] = best;
    });
    std::optional<Candidate> best;
    for (auto &b : bests) best = best_of(best, b);
    if (!best) return none;
    const srocm_feature &m = features[best->feature];
    return split_info(*ctx, hist + 2 * static_cast<size_t>(m.hist_offset), m, *best);
}

// split.rs:966-985 feature_mask
void feature_mask(const srocm_feature *features, size_t nf, double fraction, uint32_t seed, uint32_t iteration,
                  uint8_t *mask) {
    std::vector<size_t> usable;
    for (size_t f = 0; f < nf; ++f)
        if (features[f].num_bins != 0) usable.push_back(f);
    std::fill(mask, mask + nf, 0);
    if (fraction >= 1.0) {
        for (size_t f : usable) mask[f] = 1;
        return;
    }
    size_t count = std::max<size_t>(static_cast<size_t>(round_int(static_cast<double>(usable.size()) * fraction)),
                                    std::min<size_t>(usable.size(), 1));
    std::vector<std::pair<float, size_t>> keyed;
    for (size_t f : usable) keyed.emplace_back(uniform(seed, STREAM_FEATURE_FRACTION, iteration, f), f);
    std::sort(keyed.begin(), keyed.end(), [](const auto &a, const auto &b) {
        int c = total_cmp(a.first, b.first);
        if (c != 0) return c < 0;
        return a.second < b.second;
    });
    for (size_t i = 0; i < count && i < keyed.size(); ++i) mask[keyed[i].second] = 1;
}

// ---------------------------------------------------------------------------------------------------------
// tree.rs
// ---------------------------------------------------------------------------------------------------------

constexpr double ZERO_THRESHOLD = static_cast<double>(1e-35f);  // tree.rs:13
inline double nan_to_zero(double v) { return std::isnan(v) ? 0.0 : v; }
inline double round_to_zero(double v) { return std::fabs(v) > ZERO_THRESHOLD ? v : 0.0; }

struct Tree {
    size_t num_leaves = 1;
    std::vector<int32_t> split_feature;
    std::vector<float> split_gain;
    std::vector<uint32_t> threshold_bin;
    std::vector<int8_t> decision_type;
    std::vector<int32_t> left_child, right_child;
    std::vector<double> leaf_value{0.0}, leaf_weight{0.0};
    std::vector<int64_t> leaf_count{0};
    std::vector<double> internal_value, internal_weight;
    std::vector<int64_t> internal_count;
    double shrinkage = 1.0;
    std::vector<int32_t> leaf_parent{-1}, leaf_depth{0};
    // Test diagnostics, not part of silvic's tree: the f64 gain best_leaf compared when each node was committed,
    // and each leaf's pending best gain when growth stopped (-inf without a candidate split).
    std::vector<double> commit_gain, open_gain;

    struct Children {
        double left_value, right_value;
        int64_t left_count, right_count;
        double left_weight, right_weight;
        float gain;
    };

    // tree.rs:143-177
    size_t split(size_t leaf, size_t feature, uint32_t threshold, int8_t decision_type, const Children &c) {
        int32_t node = static_cast<int32_t>(num_leaves - 1);
        size_t new_leaf = num_leaves;
        int32_t parent = leaf_parent[leaf];
        if (parent >= 0) {
            if (left_child[parent] == ~static_cast<int32_t>(leaf)) left_child[parent] = node;
            else right_child[parent] = node;
        }
        split_feature.push_back(static_cast<int32_t>(feature));
        split_gain.push_back(c.gain);
        threshold_bin.push_back(threshold);
        this->decision_type.push_back(decision_type);
        left_child.push_back(~static_cast<int32_t>(leaf));
        right_child.push_back(~static_cast<int32_t>(new_leaf));
        internal_weight.push_back(leaf_weight[leaf]);
        internal_value.push_back(leaf_value[leaf]);
        internal_count.push_back(c.left_count + c.right_count);
        leaf_value[leaf] = nan_to_zero(c.left_value);
        leaf_weight[leaf] = c.left_weight;
        leaf_count[leaf] = c.left_count;
        leaf_value.push_back(nan_to_zero(c.right_value));
        leaf_weight.push_back(c.right_weight);
        leaf_count.push_back(c.right_count);
        leaf_parent[leaf] = node;
        leaf_parent.push_back(node);
        int32_t depth = leaf_depth[leaf] + 1;
        leaf_depth[leaf] = depth;
        leaf_depth.push_back(depth);
        ++num_leaves;
        return new_leaf;
    }
    // tree.rs:180-185
    void shrink(double rate) {
        for (double &v : leaf_value) v = round_to_zero(v * rate);
        for (double &v : internal_value) v = round_to_zero(v * rate);
        shrinkage *= rate;
    }
    // tree.rs:188-193
    void add_bias(double bias) {
        for (double &v : leaf_value) v = round_to_zero(v + bias);
        for (double &v : internal_value) v = round_to_zero(v + bias);
        shrinkage = 1.0;
    }
    // tree.rs:201-203
    void set_leaf_output(size_t leaf, double v) { leaf_value[leaf] = round_to_zero(v); }
};

// ---------------------------------------------------------------------------------------------------------
// The CPU backend (cpu.rs:697-935) with per-op timers (train_cpu.rs:421-484)
// ---------------------------------------------------------------------------------------------------------

using Clock = std::chrono::steady_clock;

enum Op { T_GRAD, T_QUANT, T_RESET, T_HIST, T_PART, T_SPLIT, T_SUMS, T_ADD, T_TOTAL, T_COUNT };

struct Timer {
    double *slot;
    Clock::time_point start = Clock::now();
    explicit Timer(double *s) : slot(s) {}
    ~Timer() { *slot += std::chrono::duration<double>(Clock::now() - start).count(); }
};

struct CpuBackend {
    const srocm_dataset *data = nullptr;
    std::vector<GroupLayout> layout;
    uint32_t objective = SROCM_OBJ_REGRESSION;
    double sigmoid = 1.0;
    std::vector<float> scores, grad, hess;
    std::vector<int32_t> packed;
    int64_t max_quant = 1;
    std::vector<uint32_t> partition;
    std::vector<uint8_t> used_columns;  // the feature of each used column, for the work count
    double times[T_COUNT] = {0};
    double hist_bins = 0.0;

    RankSetup rank;  // lambdarank

    void load(const srocm_dataset *d, uint32_t obj, double sig) {
        data = d;
        layout = group_layout(d);
        objective = obj;
        sigmoid = sig;
        scores.assign(d->num_rows, 0.0f);
        grad.assign(d->num_rows, 0.0f);
        hess.assign(d->num_rows, 0.0f);
        packed.assign(d->num_rows, 0);
        partition.reserve(d->num_rows);
    }
    void init_scores(double v) { std::fill(scores.begin(), scores.end(), static_cast<float>(v)); }
    std::pair<double, double> compute_gradients() {
        Timer t(&times[T_GRAD]);
        if (objective == SROCM_OBJ_LAMBDARANK) rank_gradients(rank, data, scores.data(), grad.data(), hess.data());
        else gradients(objective, sigmoid, scores.data(), data->label, data->weight, data->num_rows, grad.data(), hess.data());
        return {max_abs(grad.data(), grad.size()), max_abs(hess.data(), hess.size())};
    }
    void quantize(const srocm_quant_spec &s) {
        Timer t(&times[T_QUANT]);
        uint64_t off = data->row_offset;
        par_chunks(data->num_rows, ROW_CHUNK, [&](uint64_t, uint64_t b, uint64_t e) {
            for (uint64_t r = b; r < e; ++r) packed[r] = quantize_row(s, grad[r], hess[r], off + r);
        });
        max_quant = std::max(s.grad_max_q, s.hess_max_q);
    }
    uint32_t reset_partition(const srocm_bag &bag) {
        Timer t(&times[T_RESET]);
        partition.clear();
        uint32_t rows = static_cast<uint32_t>(data->num_rows);
        if (bag.kind == SROCM_BAG_ALL) {
            partition.resize(rows);
            par_chunks(rows, ROW_CHUNK, [&](uint64_t, uint64_t b, uint64_t e) {
                for (uint64_t i = b; i < e; ++i) partition[i] = static_cast<uint32_t>(i);
            });
        } else {
            for (uint32_t r = 0; r < rows; ++r)
                if (in_bag(bag.seed, bag.round, data->row_offset + r, bag.fraction)) partition.push_back(r);
        }
        return static_cast<uint32_t>(partition.size());
    }
    void set_histogram_features(const uint8_t *used) {
        for (auto &g : layout) g.activate(used, data->num_features);
    }
    void histogram(srocm_leaf_range leaf, double *out) {
        Timer t(&times[T_HIST]);
        if (static_cast<uint64_t>(leaf.begin) + leaf.count > partition.size()) throw std::runtime_error("leaf outside the partition");
        size_t adds = 0;
        for (auto &g : layout) adds += g.adds;
        hist_bins += static_cast<double>(leaf.count) * static_cast<double>(adds);
        histogram_quantized(data, layout, packed.data(), max_quant, partition.data() + leaf.begin, leaf.count, out);
    }
    uint32_t partition_leaf(srocm_leaf_range leaf, const srocm_bin_split &s) {
        Timer t(&times[T_PART]);
        if (static_cast<uint64_t>(leaf.begin) + leaf.count > partition.size()) throw std::runtime_error("leaf outside the partition");
        const srocm_group &g = data->groups[s.group];
        return stable_partition(partition.data() + leaf.begin, leaf.count,
                                [&](uint32_t row) { return goes_left(s, bin_at(g, row, s.column), group_bits(g) == 16); });
    }
    void leaf_sums(const std::vector<srocm_leaf_range> &leaves, float gs, float hs, std::vector<int64_t> &out) {
        Timer t(&times[T_SUMS]);
        out.assign(2 * leaves.size(), 0);
        pool().run(static_cast<int64_t>(leaves.size()), [&](int64_t l) {
            int64_t sg = 0, sh = 0;
            for (uint32_t i = leaves[l].begin; i < leaves[l].begin + leaves[l].count; ++i) {
                uint32_t row = partition[i];
                sg += to_fixed(grad[row], gs);
                sh += to_fixed(hess[row], hs);
            }
            out[2 * l] = sg;
            out[2 * l + 1] = sh;
        });
    }
    void add_tree(const std::vector<srocm_device_node> &nodes, const std::vector<float> &leaf_values) {
        Timer t(&times[T_ADD]);
        add_tree_to(data, nodes.data(), static_cast<uint32_t>(nodes.size()), leaf_values.data(),
                    static_cast<uint32_t>(leaf_values.size()), scores.data());
    }
};

// ---------------------------------------------------------------------------------------------------------
// learner.rs
// ---------------------------------------------------------------------------------------------------------

struct Leaf {
    srocm_leaf_range range{};
    LeafSums sums;
    std::vector<double> hist;  // empty: None
    bool has_hist = false;
    std::vector<uint8_t> splittable;
    std::optional<oracle_split_info> best;
};

struct GrownTree {
    Tree tree;
    std::vector<srocm_bin_split> splits;
    std::vector<srocm_leaf_range> leaves;
};

struct Learner {
    const srocm_dataset *data;
    const oracle_params *p;
    double *split_time;
    std::optional<size_t> sums_feature;

    Learner(const srocm_dataset *d, const oracle_params *params, double *st) : data(d), p(params), split_time(st) {
        for (size_t f = 0; f < d->num_features; ++f)
            if (d->features[f].num_bins != 0) {
                sums_feature = f;
                break;
            }
    }

    bool depth_allows(int32_t depth) const { return p->max_depth <= 0 || depth < p->max_depth; }  // learner.rs:178-180
    bool may_split(int32_t depth, int64_t l, int64_t r) const {                                   // learner.rs:172-175
        int64_t min_pair = 2 * p->cfg.min_data_in_leaf;
        return depth_allows(depth) && (l >= min_pair || r >= min_pair);
    }

    // learner.rs:236-246
    void find_split(Leaf &leaf, std::vector<double> &&hist, const std::vector<uint8_t> &evaluate, double gs, double hs) {
        Timer t(split_time);
        leaf.splittable.assign(data->num_features, 0);
        oracle_split_info info = find_best_split(hist.data(), data->features, data->num_features, evaluate.data(),
                                                 leaf.sums, gs, hs, &p->cfg, leaf.splittable.data());
        if (info.found) leaf.best = info;
        else leaf.best.reset();
        leaf.hist = std::move(hist);
        leaf.has_hist = true;
    }

    // learner.rs:432-452
    srocm_bin_split bin_split(const srocm_feature &m, const oracle_split_info &info) const {
        srocm_bin_split s{};
        auto set = [&](uint32_t bin) { s.left_bins[bin / 32] |= 1u << (bin % 32); };
        if (group_bits(data->groups[m.group]) == 16) {  // the numerical rule of a 2-byte feature, as goes_left reads it
            s.left_bins[0] = info.threshold;
            s.left_bins[1] = info.default_left && m.nan_bin ? m.num_bins : 0u;
        } else if (!info.categorical) {
            for (uint32_t b = 0; b <= info.threshold; ++b) set(b);
            if (info.default_left && m.kind == SROCM_BINS_NUMERICAL && m.nan_bin) set(m.num_bins - 1);
        } else {
            for (uint32_t i = 0; i < info.num_cat_bins; ++i) set(info.cat_bins[i]);
        }
        s.group = m.group;
        s.column = m.column;
        return s;
    }

    // learner.rs:418-429
    static std::optional<size_t> best_leaf(const std::vector<Leaf> &leaves) {
        std::optional<std::pair<size_t, double>> best;
        for (size_t i = 0; i < leaves.size(); ++i) {
            if (!leaves[i].best) continue;
            if (!best || leaves[i].best->gain > best->second) best = std::make_pair(i, leaves[i].best->gain);
        }
        if (best && best->second > 0.0) return best->first;
        return std::nullopt;
    }

    // learner.rs:121-169
    GrownTree grow(CpuBackend &backend, const std::vector<uint8_t> &mask, double gs, double hs, srocm_leaf_range root,
               int64_t root_count) {
        GrownTree g;
        std::vector<Leaf> leaves(1);
        leaves[0].range = root;
        leaves[0].sums.count = root_count;
        leaves[0].splittable.assign(data->num_features, 1);
        size_t bins = 2 * data->total_bins;
        if (sums_feature && may_split(0, root_count, 0)) {
            std::vector<uint8_t> root_features = mask;
            root_features[*sums_feature] = 1;
            backend.set_histogram_features(root_features.data());
            std::vector<double> hist(bins + 1, 0.0);
            backend.histogram(root, hist.data());
            const srocm_feature &m = data->features[*sums_feature];
            double sg = 0.0, sh = 0.0;
            for (uint32_t b = 0; b < m.num_bins; ++b) {  // split.rs:101-108
                sg = sg + hist[2 * (m.hist_offset + b)];
                sh = sh + hist[2 * (m.hist_offset + b) + 1];
            }
            leaves[0].sums.grad = sg;
            leaves[0].sums.hess = sh;
            find_split(leaves[0], std::move(hist), mask, gs, hs);
        }
        while (g.tree.num_leaves < p->num_leaves) {
            auto best = best_leaf(leaves);
            if (!best) break;
            split_leaf(backend, g, leaves, *best, mask, gs, hs);
        }
        for (auto &l : leaves) {
            g.leaves.push_back(l.range);
            g.tree.open_gain.push_back(l.best ? l.best->gain : -std::numeric_limits<double>::infinity());
        }
        return g;
    }

    // learner.rs:249-352
    void split_leaf(CpuBackend &backend, GrownTree &g, std::vector<Leaf> &leaves, size_t index,
                    const std::vector<uint8_t> &mask, double gs, double hs) {
        oracle_split_info info = *leaves[index].best;
        leaves[index].best.reset();
        const srocm_feature &meta = data->features[info.feature];
        srocm_bin_split bs = bin_split(meta, info);
        srocm_leaf_range parent_range = leaves[index].range;
        int64_t parent_count = leaves[index].sums.count;
        bool may_search = leaves[index].has_hist && g.tree.num_leaves + 1 < p->num_leaves &&
                          depth_allows(g.tree.leaf_depth[index] + 1);
        bool built_left = info.left.count <= info.right.count;
        std::vector<uint8_t> evaluate(data->num_features);
        for (size_t f = 0; f < data->num_features; ++f) evaluate[f] = mask[f] && leaves[index].splittable[f];
        uint32_t left_local;
        std::vector<double> built_hist;
        bool have_built = false;
        if (may_search) {
            backend.set_histogram_features(evaluate.data());
            left_local = backend.partition_leaf(parent_range, bs);
            srocm_leaf_range side = built_left ? srocm_leaf_range{parent_range.begin, left_local}
                                               : srocm_leaf_range{parent_range.begin + left_local, parent_range.count - left_local};
            built_hist.assign(2 * data->total_bins + 1, 0.0);
            backend.histogram(side, built_hist.data());
            have_built = true;
        } else {
            left_local = backend.partition_leaf(parent_range, bs);
        }
        int64_t left_count = left_local;
        int64_t right_count = parent_count - left_count;
        if (left_count <= 0 || right_count <= 0) throw std::runtime_error("split sends no rows to one side");
        Tree::Children c;
        c.left_value = info.left_output;
        c.right_value = info.right_output;
        c.left_count = left_count;
        c.right_count = right_count;
        c.left_weight = info.left.hess * hs;
        c.right_weight = info.right.hess * hs;
        c.gain = static_cast<float>(info.gain + p->cfg.min_gain_to_split);
        g.tree.commit_gain.push_back(info.gain);
        // learner.rs:459-485 apply_split: decision_type from MissingType and default_left (tree.rs:108-122)
        int8_t decision_type;
        if (info.categorical) decision_type = static_cast<int8_t>(1 | (2 << 2));
        else {
            int8_t missing = (meta.kind == SROCM_BINS_NUMERICAL && meta.nan_bin) ? 2 : 0;
            decision_type = static_cast<int8_t>((missing << 2) | (info.default_left ? 2 : 0));
        }
        size_t right_index = g.tree.split(index, info.feature, info.categorical ? 0 : info.threshold, decision_type, c);
        if (right_index != leaves.size()) throw std::runtime_error("tree numbered the new leaf unexpectedly");
        g.splits.push_back(bs);
        std::vector<double> parent_hist = std::move(leaves[index].hist);
        bool have_parent = leaves[index].has_hist;
        Leaf left, right;
        left.range = {parent_range.begin, left_local};
        left.sums = {info.left.grad, info.left.hess, left_count};
        right.range = {parent_range.begin + left_local, parent_range.count - left_local};
        right.sums = {info.right.grad, info.right.hess, right_count};
        leaves[index] = std::move(left);
        leaves.push_back(std::move(right));
        int32_t depth = g.tree.leaf_depth[index];
        bool searched = may_split(depth, left_count, right_count);
        if (have_parent && have_built && searched) {
            size_t built = built_left ? index : right_index;
            size_t other = built_left ? right_index : index;
            // learner.rs:356-371
            for (size_t i = 0; i < 2 * data->total_bins; ++i) parent_hist[i] -= built_hist[i];
            find_split(leaves[built], std::move(built_hist), evaluate, gs, hs);
            find_split(leaves[other], std::move(parent_hist), evaluate, gs, hs);
        }
    }

    // learner.rs:376-404
    void renew_leaves(CpuBackend &backend, GrownTree &g, double max_abs_grad, double max_hess) {
        float gsc = fixed_point_scale(max_abs_grad);
        float hsc = fixed_point_scale(max_hess);
        std::vector<int64_t> sums;
        backend.leaf_sums(g.leaves, gsc, hsc, sums);
        for (size_t leaf = 0; leaf < g.leaves.size(); ++leaf) {
            double sum_grad = static_cast<double>(sums[2 * leaf]) / static_cast<double>(gsc);
            double sum_hess = static_cast<double>(sums[2 * leaf + 1]) / static_cast<double>(hsc);
            double out = leaf_output(sum_grad, sum_hess, p->cfg.lambda_l1, p->cfg.lambda_l2);
            g.tree.set_leaf_output(leaf, out);
            g.tree.leaf_weight[leaf] = sum_hess;
        }
    }
};

struct Model {
    std::vector<Tree> trees;
    std::vector<std::vector<srocm_bin_split>> splits;  // per tree, per internal node: the bins that go left
    std::vector<srocm_leaf_range> leaf_ranges;  // of the last tree grown by grow_tree
    std::vector<uint32_t> partition;
    double init_score = 0.0;
    std::vector<float> scores;
    double times[T_COUNT] = {0};
    double hist_bins = 0.0;
};

// boosting.rs:83-149 train_from and boosting.rs:227-324 train_one_iter / bag / single_leaf / add
Model *train(const srocm_dataset *d, const oracle_params *p) {
    auto model = std::make_unique<Model>();
    Clock::time_point start = Clock::now();
    CpuBackend backend;
    backend.load(d, p->objective, p->sigmoid);
    if (p->objective == SROCM_OBJ_LAMBDARANK)
        backend.rank = lambdarank_setup(d, p->sigmoid, p->lambdarank_norm != 0, p->lambdarank_truncation_level,
                                        p->label_gain, p->num_label_gain);
    // objective/mod.rs:92-97: no initial score for lambdarank
    double init = p->boost_from_average && p->objective != SROCM_OBJ_LAMBDARANK
                      ? init_score(p->objective, p->sigmoid, d->label, d->weight, d->num_rows)
                      : 0.0;
    init = std::fabs(init) > K_EPSILON ? init : 0.0;
    backend.init_scores(init);
    model->init_score = init;
    std::optional<double> constant_hessian;
    if (p->objective == SROCM_OBJ_REGRESSION && d->weight == nullptr) constant_hessian = 1.0;  // objective/mod.rs:84-89
    Learner learner(d, p, &backend.times[T_SPLIT]);
    for (uint32_t iteration = 0; iteration < p->num_iterations; ++iteration) {
        auto [mg, mh] = backend.compute_gradients();
        double gs = 1.0, hs = 1.0;
        if (!p->use_quantized_grad) throw std::runtime_error("the oracle restates the quantized path only");
        srocm_quant_spec spec = quant_spec(mg, mh, constant_hessian, p->num_grad_quant_bins, p->stochastic_rounding,
                                           p->data_random_seed, iteration);
        backend.quantize(spec);
        gs = spec.grad_scale;
        hs = spec.hess_scale;
        srocm_bag bag{};
        if (p->bagging_fraction < 1.0 && p->bagging_freq > 0) {
            bag.kind = SROCM_BAG_BERNOULLI;
            bag.seed = p->bagging_seed;
            bag.round = iteration / p->bagging_freq;
            bag.fraction = p->bagging_fraction;
        }
        uint32_t local_rows = backend.reset_partition(bag);
        std::vector<uint8_t> mask(d->num_features);
        feature_mask(d->features, d->num_features, p->feature_fraction, p->feature_fraction_seed, iteration, mask.data());
        GrownTree grown = learner.grow(backend, mask, gs, hs, {0, local_rows}, local_rows);
        if (grown.tree.num_leaves == 1) {
            if (model->trees.empty()) {  // boosting.rs:303-310
                Tree t;
                t.leaf_value[0] = init;
                model->trees.push_back(t);
                model->splits.emplace_back();
            }
            break;
        }
        if (p->quant_train_renew_leaf) learner.renew_leaves(backend, grown, mg, mh);
        // boosting.rs:313-324 add
        grown.tree.shrink(p->learning_rate);
        std::vector<srocm_device_node> nodes(grown.splits.size());
        for (size_t k = 0; k < nodes.size(); ++k) {
            nodes[k].split = grown.splits[k];
            nodes[k].left = grown.tree.left_child[k];
            nodes[k].right = grown.tree.right_child[k];
        }
        std::vector<float> leaf_values(grown.tree.leaf_value.size());
        for (size_t i = 0; i < leaf_values.size(); ++i) leaf_values[i] = static_cast<float>(grown.tree.leaf_value[i]);
        if (model->trees.empty() && init != 0.0) {
            grown.tree.add_bias(init);
            for (size_t i = 0; i < leaf_values.size(); ++i)
                leaf_values[i] = static_cast<float>(grown.tree.leaf_value[i] - init);  // replay.rs:38-40
        }
        backend.add_tree(nodes, leaf_values);
        model->trees.push_back(std::move(grown.tree));
        model->splits.push_back(grown.splits);
    }
    backend.times[T_TOTAL] = std::chrono::duration<double>(Clock::now() - start).count();
    model->partition = backend.partition;  // the last tree's row order (learner.rs:121-352)
    std::copy(backend.times, backend.times + T_COUNT, model->times);
    model->hist_bins = backend.hist_bins;
    model->scores = std::move(backend.scores);
    return model.release();
}


// One tree from given gradients (learner.rs tests' `grow`, learner.rs:599-640): quantize with the maxima,
// reset the partition, grow, and renew the leaves when `renew`; no shrinkage.
Model *grow_tree(const srocm_dataset *d, const float *grad, const float *hess, const oracle_params *p, bool renew) {
    auto model = std::make_unique<Model>();
    CpuBackend backend;
    backend.load(d, SROCM_OBJ_REGRESSION, 1.0);
    std::copy(grad, grad + d->num_rows, backend.grad.begin());
    std::copy(hess, hess + d->num_rows, backend.hess.begin());
    double mg = max_abs(grad, d->num_rows), mh = max_abs(hess, d->num_rows);
    srocm_quant_spec spec = quant_spec(mg, mh, std::nullopt, p->num_grad_quant_bins, p->stochastic_rounding,
                                       p->data_random_seed, 0);
    backend.quantize(spec);
    srocm_bag bag{};
    if (p->bagging_fraction < 1.0 && p->bagging_freq > 0) {
        bag.kind = SROCM_BAG_BERNOULLI;
        bag.seed = p->bagging_seed;
        bag.round = 0;
        bag.fraction = p->bagging_fraction;
    }
    uint32_t local = backend.reset_partition(bag);
    std::vector<uint8_t> mask(d->num_features);
    feature_mask(d->features, d->num_features, p->feature_fraction, p->feature_fraction_seed, 0, mask.data());
    Learner learner(d, p, &backend.times[T_SPLIT]);
    GrownTree g = learner.grow(backend, mask, spec.grad_scale, spec.hess_scale, {0, local}, local);
    if (renew && g.tree.num_leaves > 1) learner.renew_leaves(backend, g, mg, mh);
    model->leaf_ranges = g.leaves;
    model->partition = backend.partition;
    model->trees.push_back(std::move(g.tree));
    model->splits.push_back(g.splits);
    model->scores.assign(d->num_rows, 0.0f);
    return model.release();
}

template <typename T>
void copy_out(const std::vector<T> &v, T *out) {
    if (out) std::copy(v.begin(), v.end(), out);
}

}  // namespace

// ---------------------------------------------------------------------------------------------------------
// C API
// ---------------------------------------------------------------------------------------------------------

extern "C" {

uint32_t oracle_mix32(uint32_t x) { return mix32(x); }
void oracle_mix32_n(const uint32_t *x, uint64_t n, uint32_t *out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = mix32(x[i]);
}
float oracle_uniform(uint32_t seed, uint32_t stream, uint32_t iteration, uint64_t row) {
    return uniform(seed, stream, iteration, row);
}
void oracle_quant_spec(double max_abs_grad, double max_hess, int has_constant, double constant_hessian,
                       uint32_t num_bins, int stochastic, uint32_t seed, uint32_t iteration, srocm_quant_spec *out) {
    std::optional<double> c;
    if (has_constant) c = constant_hessian;
    *out = quant_spec(max_abs_grad, max_hess, c, num_bins, stochastic != 0, seed, iteration);
}
void oracle_quantize(const srocm_quant_spec *spec, const float *grad, const float *hess, uint64_t n,
                     uint64_t row_offset, int32_t *out) {
    par_chunks(n, ROW_CHUNK, [&](uint64_t, uint64_t b, uint64_t e) {
        for (uint64_t r = b; r < e; ++r) out[r] = quantize_row(*spec, grad[r], hess[r], row_offset + r);
    });
}
void oracle_unpack(int32_t packed, int32_t *g, int32_t *h) { unpack(packed, *g, *h); }
int oracle_in_bag(uint32_t seed, uint32_t round, uint64_t row, double fraction) {
    return in_bag(seed, round, row, fraction) ? 1 : 0;
}
float oracle_fixed_point_scale(double max_abs) { return fixed_point_scale(max_abs); }
int64_t oracle_to_fixed(float value, float scale) { return to_fixed(value, scale); }

void oracle_gradients(uint32_t objective, double sigmoid, const float *scores, const float *label,
                      const float *weight, uint64_t n, float *grad, float *hess, double *max_abs_grad,
                      double *max_hess) {
    gradients(objective, sigmoid, scores, label, weight, n, grad, hess);
    if (max_abs_grad) *max_abs_grad = max_abs(grad, n);
    if (max_hess) *max_hess = max_abs(hess, n);
}
double oracle_init_score(uint32_t objective, double sigmoid, const float *label, const float *weight, uint64_t n) {
    return init_score(objective, sigmoid, label, weight, n);
}

void oracle_set_threads(int threads) { pool().resize(threads); }
int oracle_threads(void) { return pool().size(); }

void oracle_histogram(const srocm_dataset *data, const int32_t *packed, int64_t max_quant, const uint32_t *rows,
                      uint64_t count, const uint8_t *used, double *out) {
    std::vector<GroupLayout> layout = group_layout(data);
    for (auto &g : layout) g.activate(used, data->num_features);
    histogram_quantized(data, layout, packed, max_quant, rows, count, out);
}

uint32_t oracle_partition(const srocm_dataset *data, uint32_t *rows, uint64_t count, const srocm_bin_split *split) {
    const srocm_group &g = data->groups[split->group];
    return stable_partition(rows, count, [&](uint32_t row) {
        return goes_left(*split, bin_at(g, row, split->column), group_bits(g) == 16);
    });
}

void oracle_leaf_sums(const float *grad, const float *hess, const uint32_t *partition,
                      const srocm_leaf_range *leaves, uint32_t num_leaves, float grad_scale, float hess_scale,
                      int64_t *out) {
    for (uint32_t l = 0; l < num_leaves; ++l) {
        int64_t sg = 0, sh = 0;
        for (uint32_t i = leaves[l].begin; i < leaves[l].begin + leaves[l].count; ++i) {
            sg += to_fixed(grad[partition[i]], grad_scale);
            sh += to_fixed(hess[partition[i]], hess_scale);
        }
        out[2 * l] = sg;
        out[2 * l + 1] = sh;
    }
}

int oracle_add_tree(const srocm_dataset *data, const srocm_device_node *nodes, uint32_t num_nodes,
                    const float *leaf_values, uint32_t num_leaves, float *scores) {
    if (num_leaves == 0 || num_leaves != num_nodes + 1) return SROCM_ERR_DEVICE;
    try {
        add_tree_to(data, nodes, num_nodes, leaf_values, num_leaves, scores);
    } catch (const std::exception &) {
        return SROCM_ERR_DEVICE;
    }
    return SROCM_OK;
}

void oracle_find_best_split(const double *hist, const srocm_feature *features, uint32_t num_features,
                            const uint8_t *evaluate, const srocm_sums *sums, double grad_scale,
                            double hess_scale, const srocm_split_config *cfg, oracle_split_info *out,
                            uint8_t *splittable) {
    LeafSums s{sums->grad, sums->hess, sums->count};
    *out = find_best_split(hist, features, num_features, evaluate, s, grad_scale, hess_scale, cfg, splittable);
}

double oracle_leaf_gain(double g, double h, double l1, double l2) { return leaf_gain(g, h, l1, l2); }
double oracle_leaf_output(double g, double h, double l1, double l2) { return leaf_output(g, h, l1, l2); }

void oracle_feature_mask(const srocm_feature *features, uint32_t num_features, double fraction, uint32_t seed,
                         uint32_t iteration, uint8_t *mask) {
    feature_mask(features, num_features, fraction, seed, iteration, mask);
}

void oracle_lambdarank_query(const float *scores, const float *label, const float *weight, uint32_t n,
                             const double *label_gain, uint32_t num_label_gain, double inverse_max_dcg,
                             double sigmoid, int norm, uint32_t truncation_level, float *grad, float *hess) {
    RankSetup st;
    st.sigmoid = sigmoid;
    st.norm = norm != 0;
    st.truncation_level = truncation_level;
    st.label_gain.assign(label_gain, label_gain + num_label_gain);
    st.inverse_max_dcg = {inverse_max_dcg};
    rank_query(st, 0, scores, label, weight, n, grad, hess);
}

double oracle_max_dcg_at_k(uint32_t k, const float *labels, uint32_t n, const double *label_gain,
                           uint32_t num_label_gain) {
    return max_dcg_at_k(k, labels, n, std::vector<double>(label_gain, label_gain + num_label_gain));
}

double oracle_sigmoid_table_get(double sigmoid, double delta) { return sigmoid_table(sigmoid).get(delta); }

int oracle_check_labels(const float *label, uint64_t n, uint32_t num_gains) { return check_labels(label, n, num_gains); }

void oracle_lambdarank_gradients(const srocm_dataset *data, const oracle_params *p, const float *scores, float *grad,
                                 float *hess) {
    RankSetup st = lambdarank_setup(data, p->sigmoid, p->lambdarank_norm != 0, p->lambdarank_truncation_level,
                                    p->label_gain, p->num_label_gain);
    rank_gradients(st, data, scores, grad, hess);
}

void oracle_default_params(oracle_params *p) {
    std::memset(p, 0, sizeof(*p));
    p->lambdarank_norm = 1;
    p->lambdarank_truncation_level = 30;
    p->objective = SROCM_OBJ_REGRESSION;
    p->sigmoid = 1.0;
    p->num_iterations = 100;
    p->learning_rate = 0.1;
    p->num_leaves = 31;
    p->max_depth = -1;
    p->cfg.min_data_in_leaf = 20;
    p->cfg.min_sum_hessian_in_leaf = 1e-3;
    p->cfg.lambda_l1 = 0.0;
    p->cfg.lambda_l2 = 0.0;
    p->cfg.min_gain_to_split = 0.0;
    p->cfg.max_cat_to_onehot = 4;
    p->cfg.max_cat_threshold = 32;
    p->cfg.cat_l2 = 10.0;
    p->cfg.cat_smooth = 10.0;
    p->cfg.min_data_per_group = 100;
    p->bagging_fraction = 1.0;
    p->bagging_freq = 0;
    p->bagging_seed = 3;
    p->feature_fraction = 1.0;
    p->feature_fraction_seed = 2;
    p->data_random_seed = 1;
    p->num_grad_quant_bins = 4;
    p->use_quantized_grad = 1;
    p->quant_train_renew_leaf = 1;
    p->stochastic_rounding = 1;
    p->boost_from_average = 1;
}

void *oracle_train(const srocm_dataset *data, const oracle_params *params) {
    try {
        return train(data, params);
    } catch (const std::exception &) {
        return nullptr;
    }
}
void oracle_model_free(void *model) { delete static_cast<Model *>(model); }
uint32_t oracle_model_num_trees(const void *model) {
    return static_cast<uint32_t>(static_cast<const Model *>(model)->trees.size());
}
double oracle_model_init_score(const void *model) { return static_cast<const Model *>(model)->init_score; }
uint32_t oracle_model_tree_leaves(const void *model, uint32_t tree) {
    return static_cast<uint32_t>(static_cast<const Model *>(model)->trees[tree].num_leaves);
}

void oracle_model_tree(const void *model, uint32_t tree, int32_t *split_feature, uint32_t *threshold_bin,
                       int8_t *decision_type, int32_t *left_child, int32_t *right_child, float *split_gain,
                       double *internal_value, double *internal_weight, int64_t *internal_count,
                       double *leaf_value, double *leaf_weight, int64_t *leaf_count, int32_t *leaf_depth) {
    const Tree &t = static_cast<const Model *>(model)->trees[tree];
    copy_out(t.split_feature, split_feature);
    copy_out(t.threshold_bin, threshold_bin);
    copy_out(t.decision_type, decision_type);
    copy_out(t.left_child, left_child);
    copy_out(t.right_child, right_child);
    copy_out(t.split_gain, split_gain);
    copy_out(t.internal_value, internal_value);
    copy_out(t.internal_weight, internal_weight);
    copy_out(t.internal_count, internal_count);
    copy_out(t.leaf_value, leaf_value);
    copy_out(t.leaf_weight, leaf_weight);
    copy_out(t.leaf_count, leaf_count);
    copy_out(t.leaf_depth, leaf_depth);
}

void oracle_model_scores(const void *model, float *out, uint64_t n) {
    const Model *m = static_cast<const Model *>(model);
    std::copy(m->scores.begin(), m->scores.begin() + static_cast<long>(std::min<uint64_t>(n, m->scores.size())), out);
}

void oracle_model_times(const void *model, double *out9) {
    const Model *m = static_cast<const Model *>(model);
    std::copy(m->times, m->times + T_COUNT, out9);
}

void *oracle_grow_tree(const srocm_dataset *data, const float *grad, const float *hess, const oracle_params *params,
                       int renew) {
    try {
        return grow_tree(data, grad, hess, params, renew != 0);
    } catch (const std::exception &) {
        return nullptr;
    }
}

void oracle_model_leaf_ranges(const void *model, srocm_leaf_range *out) {
    const Model *m = static_cast<const Model *>(model);
    std::copy(m->leaf_ranges.begin(), m->leaf_ranges.end(), out);
}

void oracle_model_partition(const void *model, uint32_t *out) {
    const Model *m = static_cast<const Model *>(model);
    std::copy(m->partition.begin(), m->partition.end(), out);
}

double oracle_model_hist_bins(const void *model) { return static_cast<const Model *>(model)->hist_bins; }

void oracle_model_tree_gains(const void *model, uint32_t tree, double *commit_gain, double *open_gain) {
    const Tree &t = static_cast<const Model *>(model)->trees[tree];
    copy_out(t.commit_gain, commit_gain);
    copy_out(t.open_gain, open_gain);
}

void oracle_model_tree_left_bins(const void *model, uint32_t tree, uint32_t *out) {
    const Model *m = static_cast<const Model *>(model);
    const auto &sp = m->splits.at(tree);
    for (size_t k = 0; k < sp.size(); ++k) std::copy(sp[k].left_bins, sp[k].left_bins + 8, out + 8 * k);
}

}  // extern "C"
