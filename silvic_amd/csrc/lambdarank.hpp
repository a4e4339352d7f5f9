// lambdarank.hpp - LambdaRank-NDCG gradients on the host, in f64, as silvic's CPU backend computes them
// (crates/silvic-core/src/objective/lambdarank.rs:190-420: LightGBM 3.3.5 `GetGradientsForOneQuery` with f64
// accumulation, then the f32 store and the row weight).
//
// Per query: the rows are ranked by score, descending, ties by row (lambdarank.rs:142-170); every pair of ranks
// (i, j) with i below the truncation level, j > i and different labels adds its lambda and hessian to both items,
// i's row of pairs in j order after what the earlier rows added to i (lambdarank.rs:355-400); the sums are scaled by
// log2(1 + s) / s of the query's lambda sum s when normalizing (lambdarank.rs:287-300). The pair probability comes
// from LightGBM's 2^20-entry sigmoid table (lambdarank.rs:44-116) and the discounts 1 / log2(2 + rank) from its
// 10,000-entry table (lambdarank.rs:30-43); both are built here with the C library's exp and log2, as the reference
// builds them with Rust's f64::exp / f64::log2 on the same host. Queries run in parallel on host threads; a
// query's result depends only on its own rows, so the thread count changes nothing.
#pragma once

#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <limits>
#include <mutex>
#include <thread>
#include <vector>

#ifdef __HIPCC__
#define SRANK_HD __host__ __device__
#else
#define SRANK_HD
#endif

namespace srocm_rank {

constexpr size_t SIGMOID_BINS = size_t(1) << 20;    // lambdarank.rs:28
constexpr double MIN_SIGMOID_INPUT = -50.0;          // lambdarank.rs:25
constexpr size_t DISCOUNT_TABLE = 10000;             // lambdarank.rs:22 (kMaxPosition)
constexpr double DISTANCE_EPSILON = static_cast<double>(0.01f);  // lambdarank.rs:31
constexpr size_t QUERIES_PER_CLAIM = 16;             // queries a thread takes at a time

struct Setup {
    double sigmoid = 1.0;
    bool norm = true;
    uint32_t truncation_level = 30;
    std::vector<double> label_gain;
    std::vector<double> inverse_max_dcg;  // per query
    std::vector<uint32_t> boundaries;     // num_queries + 1
};

// A label as Rust's `as` casts convert it (lambdarank.rs:172-188, :349): NaN to 0, values outside the target's range
// to its nearest end, the rest truncated toward zero. A NaN label passes silvic's checks and takes label 0's gain.
SRANK_HD inline int32_t label_as_i32(float l) {
    if (!(l == l)) return 0;
    if (l <= -2147483648.0f) return INT32_MIN;
    if (l >= 2147483648.0f) return INT32_MAX;
    return static_cast<int32_t>(l);
}
SRANK_HD inline uint64_t label_as_index(float l) {
    if (!(l > 0.0f)) return 0;  // NaN, zero and negative labels
    if (l >= 18446744073709551616.0f) return UINT64_MAX;
    return static_cast<uint64_t>(l);
}

// Host threads started once that run one job at a time: run(fn) calls fn(w) on every worker w in 0 .. size() - 1,
// the calling thread being worker 0, and returns when every call has returned. Workers sleep between jobs, so a job
// costs one wake-up instead of starting threads.
class WorkPool {
public:
    explicit WorkPool(unsigned threads) : n_(std::max(1u, threads)) {
        for (unsigned w = 1; w < n_; ++w) threads_.emplace_back([this, w] { loop(w); });
    }
    ~WorkPool() {
        {
            std::lock_guard<std::mutex> lock(mu_);
            stop_ = true;
        }
        start_.notify_all();
        for (auto &t : threads_) t.join();
    }
    WorkPool(const WorkPool &) = delete;
    WorkPool &operator=(const WorkPool &) = delete;
    unsigned size() const { return n_; }
    void run(const std::function<void(unsigned)> &fn) {
        {
            std::lock_guard<std::mutex> lock(mu_);
            job_ = &fn;
            pending_ = n_ - 1;
            ++gen_;
        }
        start_.notify_all();
        fn(0);
        std::unique_lock<std::mutex> lock(mu_);
        done_.wait(lock, [this] { return pending_ == 0; });
        job_ = nullptr;
    }

private:
    void loop(unsigned w) {
        uint64_t seen = 0;
        for (;;) {
            const std::function<void(unsigned)> *job;
            {
                std::unique_lock<std::mutex> lock(mu_);
                start_.wait(lock, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
                job = job_;
            }
            (*job)(w);
            std::lock_guard<std::mutex> lock(mu_);
            if (--pending_ == 0) done_.notify_one();
        }
    }
    const unsigned n_;
    std::vector<std::thread> threads_;
    std::mutex mu_;
    std::condition_variable start_, done_;
    const std::function<void(unsigned)> *job_ = nullptr;
    uint64_t gen_ = 0;
    unsigned pending_ = 0;
    bool stop_ = false;
};

// The normalization factor of a query with lambda sum s (lambdarank.rs:287-300): log2(1 + s) / s when normalizing
// and s > 0, else 1; the C library's log2, as silvic's f64::log2.
inline double norm_factor(bool norm, double s) { return norm && s > 0.0 ? std::log2(1.0 + s) / s : 1.0; }

// A key whose ascending order is the score's descending order; +0.0f folds -0 into 0 (equal under `>`).
SRANK_HD inline uint32_t rank_key(float score) {
    float s = score + 0.0f;
    uint32_t bits;
    __builtin_memcpy(&bits, &s, 4);
    const uint32_t ascending = (bits >> 31) ? ~bits : (bits | 0x80000000u);
    return ~ascending;
}

// The bin of LightGBM's sigmoid table a score difference takes (lambdarank.rs:96-116): the clamped ends, else the bin
// of (delta - min_input) * idx_factor truncated, at most the last. The reference's cast saturates: a product at or
// above the last bin takes the last, a NaN or negative one bin 0; in between the truncation fits 32 bits. Shared by
// the host and the device, so both take the same f64 operations.
SRANK_HD inline uint32_t table_bin(double min_input, double max_input, double idx_factor, double delta) {
    constexpr uint32_t last = static_cast<uint32_t>(SIGMOID_BINS - 1);
    if (delta <= min_input) return 0;
    if (delta >= max_input) return last;
    const double x = (delta - min_input) * idx_factor;
    return x >= static_cast<double>(last) ? last : (x > 0.0 ? static_cast<uint32_t>(x) : 0u);
}

// One pair (i above j in the ranking, different labels) as lambdarank.rs:355-400 adds it: the sign, the lambda term
// p_lambda and the hessian term. In two parts around the table read, so the device can have the reads of a row in
// flight while it adds up the row before; the host takes both parts at once (pair_term). Shared by the host and the
// device.
struct PairTerm {
    double sign, p_lambda, p_hessian;
};
struct PairPrep {
    double sign, delta_ndcg;
    uint32_t bin;  // of the sigmoid table
};
SRANK_HD inline PairPrep pair_prep(double si, float li, double gi, double di, double sj, float lj, double gj, double dj,
                                   double inv_max_dcg, bool by_distance, double min_input, double max_input,
                                   double idx_factor) {
    PairPrep q;
    q.sign = li > lj ? 1.0 : -1.0;
    const double delta_score = q.sign * (si - sj);
    const double dcg_gap = q.sign * (gi - gj);
    const double paired_discount = fabs(di - dj);
    q.delta_ndcg = dcg_gap * paired_discount * inv_max_dcg;
    if (by_distance) q.delta_ndcg /= DISTANCE_EPSILON + fabs(delta_score);
    q.bin = table_bin(min_input, max_input, idx_factor, delta_score);
    return q;
}
SRANK_HD inline PairTerm pair_finish(const PairPrep &q, double p, double sigmoid, double sigmoid2) {
    PairTerm t;
    t.sign = q.sign;
    t.p_lambda = p * (-sigmoid * q.delta_ndcg);
    t.p_hessian = p * (1.0 - p) * (sigmoid2 * q.delta_ndcg);
    return t;
}
SRANK_HD inline PairTerm pair_term(double si, float li, double gi, double di, double sj, float lj, double gj, double dj,
                                   double inv_max_dcg, bool by_distance, double sigmoid, double sigmoid2,
                                   const double *table, double min_input, double max_input, double idx_factor) {
    const PairPrep q = pair_prep(si, li, gi, di, sj, lj, gj, dj, inv_max_dcg, by_distance, min_input, max_input,
                                 idx_factor);
    return pair_finish(q, table[q.bin], sigmoid, sigmoid2);
}

class Ranker {
public:
    void configure(Setup s) {
        setup_ = std::move(s);
        if (table_.empty() || table_sigmoid_ != setup_.sigmoid) build_table(setup_.sigmoid);
        if (discount_.empty()) {
            discount_.resize(DISCOUNT_TABLE);
            for (size_t i = 0; i < DISCOUNT_TABLE; ++i) discount_[i] = 1.0 / std::log2(2.0 + static_cast<double>(i));
        }
    }

    const Setup &setup() const { return setup_; }
    const std::vector<double> &sigmoid_table() const { return table_; }
    const std::vector<double> &discounts() const { return discount_; }
    double min_input() const { return min_input_; }
    double max_input() const { return max_input_; }
    double idx_factor() const { return idx_factor_; }

    // DCG of the best ordering of a query's labels, truncated at k (lambdarank.rs:119-139): the labels in
    // descending order, each weighted by its rank's discount, summed in rank order.
    double max_dcg_at_k(size_t k, const float *labels, size_t n) const {
        std::vector<size_t> count(setup_.label_gain.size(), 0);
        for (size_t i = 0; i < n; ++i) count[label_as_index(labels[i])] += 1;
        size_t top = count.size() - 1;
        double dcg = 0.0;
        for (size_t j = 0; j < std::min(k, n); ++j) {
            while (top > 0 && count[top] == 0) --top;
            dcg += discount(j) * setup_.label_gain[top];
            count[top] -= 1;
        }
        return dcg;
    }

    // objective/mod.rs:39-55: 1 / max DCG of each query at the truncation level, 0 for a query without gain
    void derive_inverse_max_dcg(const float *label) {
        const size_t nq = setup_.boundaries.size() - 1;
        setup_.inverse_max_dcg.resize(nq);
        for (size_t q = 0; q < nq; ++q) {
            const size_t b = setup_.boundaries[q], e = setup_.boundaries[q + 1];
            const double m = max_dcg_at_k(setup_.truncation_level, label + b, e - b);
            setup_.inverse_max_dcg[q] = m > 0.0 ? 1.0 / m : 0.0;
        }
    }

    // grad/hess of the rows of the listed queries (every query when `queries` is null: nq of them) from scores,
    // labels and optional weights, the queries shared out over the pool's threads.
    void gradients(const uint32_t *queries, size_t nq, const float *scores, const float *label, const float *weight,
                   float *grad, float *hess, WorkPool &pool) const {
        std::atomic<size_t> next{0};
        pool.run([&](unsigned) {
            Scratch sc;
            for (;;) {
                const size_t q0 = next.fetch_add(QUERIES_PER_CLAIM);
                if (q0 >= nq) break;
                const size_t q1 = std::min(nq, q0 + QUERIES_PER_CLAIM);
                for (size_t k = q0; k < q1; ++k) one_query(queries ? queries[k] : k, scores, label, weight, grad, hess, sc);
            }
        });
    }

private:
    struct Scratch {
        std::vector<uint64_t> keys;
        std::vector<uint32_t> row;      // local row of each rank
        std::vector<double> score, gain, disc, lambda, hessian;
        std::vector<float> lab;
    };

    Setup setup_;
    std::vector<double> table_, discount_;
    double table_sigmoid_ = 0.0, min_input_ = 0.0, max_input_ = 0.0, idx_factor_ = 0.0;

    // LightGBM's sigmoid table: 1 / (1 + exp(sigmoid * x)) at the lower edge of each bin over [-50, 50] / sigmoid / 2
    void build_table(double sigmoid) {
        min_input_ = MIN_SIGMOID_INPUT / sigmoid / 2.0;
        max_input_ = -min_input_;
        idx_factor_ = static_cast<double>(SIGMOID_BINS) / (max_input_ - min_input_);
        table_.resize(SIGMOID_BINS);
        for (size_t i = 0; i < SIGMOID_BINS; ++i) {
            const double x = static_cast<double>(i) / idx_factor_ + min_input_;
            table_[i] = 1.0 / (1.0 + std::exp(x * sigmoid));
        }
        table_sigmoid_ = sigmoid;
    }

    double discount(size_t rank) const {
        return rank < DISCOUNT_TABLE ? discount_[rank] : 1.0 / std::log2(2.0 + static_cast<double>(rank));
    }

    void one_query(size_t q, const float *scores, const float *label, const float *weight, float *grad, float *hess,
                   Scratch &sc) const {
        const size_t b = setup_.boundaries[q], n = setup_.boundaries[q + 1] - b;
        if (n == 0) return;
        sc.keys.resize(n);
        for (size_t r = 0; r < n; ++r) sc.keys[r] = (static_cast<uint64_t>(rank_key(scores[b + r])) << 32) | r;
        std::sort(sc.keys.begin(), sc.keys.end());
        sc.row.resize(n);
        sc.score.resize(n);
        sc.lab.resize(n);
        sc.gain.resize(n);
        sc.disc.resize(n);
        sc.lambda.assign(n, 0.0);
        sc.hessian.assign(n, 0.0);
        for (size_t k = 0; k < n; ++k) {
            const uint32_t r = static_cast<uint32_t>(sc.keys[k] & 0xffffffffu);
            sc.row[k] = r;
            sc.score[k] = static_cast<double>(scores[b + r]);
            sc.lab[k] = label[b + r];
            sc.gain[k] = setup_.label_gain[label_as_index(sc.lab[k])];
            sc.disc[k] = discount(k);
        }
        // -inf scores rank last; the lowest score skips one trailing -inf (lambdarank.rs:333-340)
        size_t valid = n;
        for (size_t k = 0; k < n; ++k)
            if (sc.score[k] == -std::numeric_limits<double>::infinity()) {
                valid = k;
                break;
            }
        size_t worst = n - 1;
        if (worst > 0 && sc.score[worst] == -std::numeric_limits<double>::infinity()) --worst;
        const double sigmoid = setup_.sigmoid, sigmoid2 = sigmoid * sigmoid;
        const double inv_max_dcg = setup_.inverse_max_dcg[q];
        const bool by_distance = setup_.norm && sc.score[0] != sc.score[worst];
        const size_t rows_i = std::min<size_t>(setup_.truncation_level, valid > 0 ? valid - 1 : 0);
        double sum_lambdas = 0.0;
        for (size_t i = 0; i < rows_i; ++i) {
            const double si = sc.score[i], gi = sc.gain[i], di = sc.disc[i];
            const float li = sc.lab[i];
            double lam_i = sc.lambda[i], hes_i = sc.hessian[i];
            for (size_t j = i + 1; j < valid; ++j) {
                if (sc.lab[j] == li) continue;
                const PairTerm t = pair_term(si, li, gi, di, sc.score[j], sc.lab[j], sc.gain[j], sc.disc[j], inv_max_dcg,
                                             by_distance, sigmoid, sigmoid2, table_.data(), min_input_, max_input_,
                                             idx_factor_);
                lam_i += t.sign * t.p_lambda;
                sc.lambda[j] -= t.sign * t.p_lambda;
                hes_i += t.p_hessian;
                sc.hessian[j] += t.p_hessian;
                sum_lambdas -= 2.0 * t.p_lambda;
            }
            sc.lambda[i] = lam_i;
            sc.hessian[i] = hes_i;
        }
        const double factor = norm_factor(setup_.norm, sum_lambdas);
        for (size_t k = 0; k < n; ++k) {
            const size_t row = b + sc.row[k];
            float g = static_cast<float>(sc.lambda[k] * factor);
            float h = static_cast<float>(sc.hessian[k] * factor);
            if (weight) {
                g *= weight[row];
                h *= weight[row];
            }
            grad[row] = g;
            hess[row] = h;
        }
    }
};

}  // namespace srocm_rank
