/*
 * silvic_oracle.h - the oracle: a CPU restatement of silvic's quantized training path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP backend is compared with and the CPU
 * baseline `bench.py` times; only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s cpu_baseline leg load
 * it. The product library (silvic_amd/_lib/libsilvic_rocm.so) never links, loads or calls it.
 *
 * Every function follows the reference file:line named beside it, operation for operation wherever floating
 * point is involved (built with -ffp-contract=off and no fast math, as Rust compiles f64 arithmetic).
 *
 * Pinning (how each part is checked beyond restating it; the tests name the reference test they port):
 *   quantize            closed forms + the reference's unit invariants (quantize.rs:167-216)
 *   histogram           brute-force direct sums (cpu.rs:1000-1090), exact integers
 *   stable partition    filter-left-then-right closed form (cpu.rs:1092-1121)
 *   leaf_sums/add_tree  direct sums and the reference's two-leaf case (cpu.rs:1123-1179)
 *   find_best_split     brute force over every candidate (split.rs:1070-1489), tie and constraint cases
 *   feature_mask        the LightGBM count cases (split.rs:1491-1506)
 *   learner             -G/H leaves and partition/leaf consistency (learner.rs:657-740)
 *   tree arrays         LightGBM node numbering case (tree.rs:250-273)
 *   gradients (binary)  parity unpinned beyond "same glibc exp": no reference vector fixes its bits
 *                       (crates/silvic-serve/README.md:85-86 notes exp may differ in its last bit)
 *   exact f64 bits of split gains: the reference pins them only to 1e-9 (split.rs:1102-1107); bit
 *                       equality of this restatement with silvic is otherwise unpinned.
 */
#ifndef SILVIC_ORACLE_H
#define SILVIC_ORACLE_H

#include "../include/silvic_rocm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* quantize.rs:14-31 */
uint32_t oracle_mix32(uint32_t x);
/* mix32 over an array (test helper). */
void oracle_mix32_n(const uint32_t *x, uint64_t n, uint32_t *out);
float oracle_uniform(uint32_t seed, uint32_t stream, uint32_t iteration, uint64_t row);
/* quantize.rs:56-84; has_constant selects Some(constant_hessian) */
void oracle_quant_spec(double max_abs_grad, double max_hess, int has_constant, double constant_hessian,
                       uint32_t num_bins, int stochastic, uint32_t seed, uint32_t iteration, srocm_quant_spec *out);
/* quantize.rs:100-136, cpu.rs:782-800 */
void oracle_quantize(const srocm_quant_spec *spec, const float *grad, const float *hess, uint64_t n,
                     uint64_t row_offset, int32_t *out);
/* quantize.rs:140-143 */
void oracle_unpack(int32_t packed, int32_t *g, int32_t *h);
/* quantize.rs:147-149 */
int oracle_in_bag(uint32_t seed, uint32_t round, uint64_t row, double fraction);
/* quantize.rs:153-165 */
float oracle_fixed_point_scale(double max_abs);
int64_t oracle_to_fixed(float value, float scale);

/* objective/{binary,regression}.rs gradients; returns maxima as cpu.rs:774-778 */
void oracle_gradients(uint32_t objective, double sigmoid, const float *scores, const float *label,
                      const float *weight, uint64_t n, float *grad, float *hess, double *max_abs_grad,
                      double *max_hess);
/* objective/mod.rs:92-109 (boost_from_average on) */
double oracle_init_score(uint32_t objective, double sigmoid, const float *label, const float *weight, uint64_t n);

/* Threads of the oracle's pool (0: hardware_concurrency). */
void oracle_set_threads(int threads);
int oracle_threads(void);

/* cpu.rs:479-513 histogram_quantized over rows[0..count]; `used` (one byte per feature, or NULL for all)
 * selects columns as GroupLayout::activate (cpu.rs:69-98). out: 2 * total_bins doubles. */
void oracle_histogram(const srocm_dataset *data, const int32_t *packed, int64_t max_quant, const uint32_t *rows,
                      uint64_t count, const uint8_t *used, double *out);
/* cpu.rs:556-599 stable_partition by a BinSplit on the rows in place; returns the left count. */
uint32_t oracle_partition(const srocm_dataset *data, uint32_t *rows, uint64_t count, const srocm_bin_split *split);
/* cpu.rs:886-908 */
void oracle_leaf_sums(const float *grad, const float *hess, const uint32_t *partition,
                      const srocm_leaf_range *leaves, uint32_t num_leaves, float grad_scale, float hess_scale,
                      int64_t *out);
/* cpu.rs:666-695 add_tree_to */
int oracle_add_tree(const srocm_dataset *data, const srocm_device_node *nodes, uint32_t num_nodes,
                    const float *leaf_values, uint32_t num_leaves, float *scores);

/* split.rs SplitInfo with the rule spelled out: numerical (threshold, default_left) or categorical bins. */
typedef struct oracle_split_info {
    int32_t found;
    int32_t feature;
    double gain;
    int32_t categorical;
    uint32_t threshold;
    uint32_t default_left;
    uint32_t num_cat_bins;
    uint32_t cat_bins[256];
    srocm_sums left;
    srocm_sums right;
    double left_output;
    double right_output;
} oracle_split_info;

/* split.rs:919-961 find_best_split */
void oracle_find_best_split(const double *hist, const srocm_feature *features, uint32_t num_features,
                            const uint8_t *evaluate, const srocm_sums *sums, double grad_scale,
                            double hess_scale, const srocm_split_config *cfg, oracle_split_info *out,
                            uint8_t *splittable);
/* split.rs:159-162, 190-192 */
double oracle_leaf_gain(double g, double h, double l1, double l2);
double oracle_leaf_output(double g, double h, double l1, double l2);
/* split.rs:966-985 */
void oracle_feature_mask(const srocm_feature *features, uint32_t num_features, double fraction, uint32_t seed,
                         uint32_t iteration, uint8_t *mask);

/* Training parameters the path reads (config.rs:123-167 defaults). */
typedef struct oracle_params {
    uint32_t objective;            /* SROCM_OBJ_REGRESSION / SROCM_OBJ_BINARY / SROCM_OBJ_LAMBDARANK */
    double sigmoid;
    uint32_t num_iterations;
    double learning_rate;
    uint32_t num_leaves;
    int32_t max_depth;
    srocm_split_config cfg;
    double bagging_fraction;
    uint32_t bagging_freq;
    uint32_t bagging_seed;
    double feature_fraction;
    uint32_t feature_fraction_seed;
    uint32_t data_random_seed;
    uint32_t num_grad_quant_bins;
    uint8_t use_quantized_grad;
    uint8_t quant_train_renew_leaf;
    uint8_t stochastic_rounding;
    uint8_t boost_from_average;
    /* lambdarank (config.rs:101-103, 152-154); label_gain NULL: LightGBM's default 2^i - 1, i < 31 */
    uint32_t lambdarank_norm;
    uint32_t lambdarank_truncation_level;
    const double *label_gain;
    uint32_t num_label_gain;
} oracle_params;

void oracle_default_params(oracle_params *p);

/* LambdarankNDCG for one query (objective/lambdarank.rs:254-301) with a given inverse max DCG; grad/hess hold n. */
void oracle_lambdarank_query(const float *scores, const float *label, const float *weight, uint32_t n,
                             const double *label_gain, uint32_t num_label_gain, double inverse_max_dcg,
                             double sigmoid, int norm, uint32_t truncation_level, float *grad, float *hess);
/* lambdarank.rs:119-139 */
// lambdarank.rs:172-188 check_labels (Rust's saturating casts: a NaN label passes as label 0)
int oracle_check_labels(const float *label, uint64_t n, uint32_t num_gains);
double oracle_max_dcg_at_k(uint32_t k, const float *labels, uint32_t n, const double *label_gain,
                           uint32_t num_label_gain);
/* lambdarank.rs:104-116 SigmoidTable::get */
double oracle_sigmoid_table_get(double sigmoid, double delta);
/* Every query's gradients of a dataset with query boundaries (lambdarank.rs:190-246, setup objective/mod.rs:34-62). */
void oracle_lambdarank_gradients(const srocm_dataset *data, const oracle_params *params, const float *scores,
                                 float *grad, float *hess);

/* boosting.rs:83-149 train_from (no init model, no validation sets). Returns a model handle. */
void *oracle_train(const srocm_dataset *data, const oracle_params *params);
void oracle_model_free(void *model);
uint32_t oracle_model_num_trees(const void *model);
double oracle_model_init_score(const void *model);
uint32_t oracle_model_tree_leaves(const void *model, uint32_t tree);
/* Copies tree `tree`'s arrays; every pointer may be NULL. Node arrays hold num_leaves-1 entries, leaf arrays
 * num_leaves. decision_type is LightGBM's (tree.rs:8-21). */
void oracle_model_tree(const void *model, uint32_t tree, int32_t *split_feature, uint32_t *threshold_bin,
                       int8_t *decision_type, int32_t *left_child, int32_t *right_child, float *split_gain,
                       double *internal_value, double *internal_weight, int64_t *internal_count,
                       double *leaf_value, double *leaf_weight, int64_t *leaf_count, int32_t *leaf_depth);
/* The training scores after the last tree. */
void oracle_model_scores(const void *model, float *out, uint64_t n);
/* Seconds spent per op (Timed wrapper, crates/silvic-core/tests/train_cpu.rs:421-484): gradients, quantize,
 * reset_partition, histogram, partition, split search, leaf_sums, add_tree, total. */
void oracle_model_times(const void *model, double *out9);
/* One tree grown from given gradients, quantized with their maxima (seed data_random_seed, iteration 0),
 * leaves renewed when `renew` (learner.rs tests, learner.rs:599-640). Not shrunk. */
void *oracle_grow_tree(const srocm_dataset *data, const float *grad, const float *hess, const oracle_params *params,
                       int renew);
/* The leaf row ranges and the partition after oracle_grow_tree. */
void oracle_model_leaf_ranges(const void *model, srocm_leaf_range *out);
void oracle_model_partition(const void *model, uint32_t *out);
/* Sum over histogram builds of rows x used feature columns (the "bins" work unit). */
double oracle_model_hist_bins(const void *model);
/* Test diagnostics of tree `tree`: per internal node the f64 gain best_leaf compared when it was committed
 * (num_leaves-1 entries), per leaf its pending best gain when growth stopped (num_leaves entries; -inf without a
 * candidate). Either pointer may be NULL. */
void oracle_model_tree_gains(const void *model, uint32_t tree, double *commit_gain, double *open_gain);
/* per internal node of tree `tree`, 8 words: the bins that go left (the BinSplit the learner handed the backend) */
void oracle_model_tree_left_bins(const void *model, uint32_t tree, uint32_t *out);

#ifdef __cplusplus
}
#endif

#endif
