/*
 * silvic_rocm.h - C ABI of the MI355X (gfx950) training backend for silvic's quantized-gradient
 * histogram / split path.
 *
 * The entry points mirror silvic-core's `trait Backend` (crates/silvic-core/src/backend/mod.rs:115-179)
 * one to one, so a thin Rust crate (`silvic-rocm`, shaped like crates/silvic-neuron/src/training.rs:324)
 * can implement `Backend` by calling them. On top of the trait mirror there is a device-side extension
 * (sibling subtraction, best-split search and whole-tree growth) that is valid only when the collective is
 * local (one rank), the case a single GPU covers.
 *
 * Conventions (crates/silvic-core/src/error.rs:5-70; crates/silvic-gpu/src/cuda.rs:19-54):
 *   - Every call returns an `int` status: SROCM_OK (0) or one of the SROCM_ERR_* kinds, which are
 *     `SilvicError::kind()`. The message of the last failure is `srocm_last_error(ctx)`.
 *   - No call aborts the process and no C++ exception crosses this boundary; a missing driver or device
 *     is an error (SROCM_ERR_DEVICE), never a crash.
 *   - Host pointers belong to the caller and are only read or written for the duration of the call.
 *   - One caller at a time per context (the trait's methods take `&mut self`); a context may move between
 *     threads.
 *   - Every histogram a backend returns in quantized mode holds exact integers, so it equals the CPU
 *     backend's bit for bit.
 */
#ifndef SILVIC_ROCM_H
#define SILVIC_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: SilvicError::kind() (crates/silvic-core/src/error.rs:33-45) ---------------------- */
enum {
    SROCM_OK = 0,
    SROCM_ERR_CONFIG = 1,
    SROCM_ERR_DATA = 2,
    SROCM_ERR_DEVICE = 3,
    SROCM_ERR_COLLECTIVE = 4,
    SROCM_ERR_MODEL = 5,
    SROCM_ERR_UNSUPPORTED = 6,
    SROCM_ERR_INTERRUPTED = 7,
    SROCM_ERR_INTERNAL = 8
};

/* ---- plain-C mirrors of the reference's value types --------------------------------------------------- */

/* BinMapper variant of a feature (crates/silvic-core/src/data/bin_mapper.rs:25-40). */
enum { SROCM_BINS_TRIVIAL = 0, SROCM_BINS_NUMERICAL = 1, SROCM_BINS_CATEGORICAL = 2 };

/* FeatureMeta (crates/silvic-core/src/data/mod.rs:24-36) without the name and the real-valued bounds, which
 * the device never reads. */
typedef struct srocm_feature {
    uint32_t num_bins;    /* bins in the histogram, the NaN bin included; 0 for a trivial feature */
    uint32_t group;       /* the feature's group */
    uint32_t column;      /* byte offset of the feature in its group's row */
    uint32_t hist_offset; /* index of the feature's bin 0 in the flat histogram */
    uint32_t kind;        /* SROCM_BINS_* */
    uint32_t nan_bin;     /* numerical: 1 when bin num_bins-1 holds NaN (MissingType::NaN) */
} srocm_feature;

/* FeatureGroup (crates/silvic-core/src/data/mod.rs:48-59), plus `bin_bits`, an extension the reference does not
 * have (its bins are always bytes, and it rejects max_bin > 255, config.rs:407-412):
 *   0 or 8: silvic's byte bins, data[row * row_stride + column];
 *   16: numerical features of up to 1024 bins, each bin a little-endian u16 at byte offset `column` of the row;
 *   4:  features of up to 16 bins, two to a byte: `column` counts 4-bit slots, slot c is the low half of byte c / 2
 *       when c is even, the high half when it is odd.
 * A split on a feature of a 16-bit group (srocm_bin_split, srocm_device_node, srocm_grown_tree.left_bins) encodes its
 * numerical rule in place of the 256-bit mask: left_bins[0] is the threshold (bins 0..=threshold go left),
 * left_bins[1] is the NaN bin + 1 when missing values go left (0 otherwise), the other words are 0. */
typedef struct srocm_group {
    uint32_t row_stride;      /* bytes per row, the feature bytes rounded up to 4 */
    uint32_t hist_offset;     /* index of the group's first bin in the flat histogram */
    uint32_t total_bins;
    uint32_t num_features;
    const uint32_t *features; /* indices into the dataset's features, in column order */
    const uint8_t *data;      /* row-major bins: data[row * row_stride + column] */
    uint32_t bin_bits;        /* 0 or 8: u8 bins; 16: u16 bins; 4: two bins a byte (extensions) */
} srocm_group;

/* BinnedDataset (crates/silvic-core/src/data/mod.rs:61-74). */
typedef struct srocm_dataset {
    uint64_t num_rows;
    uint64_t row_offset;                /* global id of local row 0; keys quantization and bagging draws */
    uint32_t num_features;
    uint32_t num_groups;
    const srocm_feature *features;      /* every input feature in input order, trivial ones included */
    const srocm_group *groups;
    uint64_t total_bins;
    const float *label;                 /* num_rows */
    const float *weight;                /* num_rows, or NULL */
    const uint32_t *query_boundaries;   /* num_queries + 1, or NULL */
    uint32_t num_queries;
} srocm_dataset;

/* ObjectiveSetup (crates/silvic-core/src/backend/mod.rs:56-71), the fields of its LambdaRank variant included.
 * Lambdarank gradients (objective/lambdarank.rs:190-420) are computed by srocm_compute_gradients and by the
 * boosting loop, bit-identical to silvic's f64 CPU path either way: on the device (k_rank_pairs) for queries of at
 * most 512 rows, on the library's host threads in f64 for longer ones. The normalization factor log2(1 + s) / s
 * of a device query is made on the device from the two doubles around log2(1 + s), one of which is the C library's;
 * when some row's f32 gradient could depend on which, the gradients are made again with the host's factors (the
 * boosting loop then takes that iteration again; nothing of the first attempt reaches the scores). They need the
 * training set's query_boundaries. */
enum { SROCM_OBJ_REGRESSION = 0, SROCM_OBJ_BINARY = 1, SROCM_OBJ_LAMBDARANK = 2 };
typedef struct srocm_objective {
    uint32_t kind;                  /* SROCM_OBJ_* */
    double sigmoid;                 /* binary and lambdarank */
    uint32_t norm;                  /* lambdarank: lambdarank_norm */
    uint32_t truncation_level;      /* lambdarank: lambdarank_truncation_level */
    const double *label_gain;       /* lambdarank: gain of each label value */
    uint32_t num_label_gain;
    const double *inverse_max_dcg;  /* lambdarank: per training query (the training set's num_queries), or NULL
                                     * for the backend to derive them from the labels as objective/mod.rs:39-55 */
} srocm_objective;

/* QuantSpec (crates/silvic-core/src/quantize.rs:33-51). */
typedef struct srocm_quant_spec {
    float inv_grad_scale;
    float inv_hess_scale;
    double grad_scale;
    double hess_scale;
    int32_t grad_max_q;
    int32_t hess_max_q;
    uint8_t constant_hessian;
    uint8_t stochastic;
    uint8_t pad_[2];
    uint32_t seed;
    uint32_t iteration;
} srocm_quant_spec;

/* BagSpec (crates/silvic-core/src/backend/mod.rs:80-90). */
enum { SROCM_BAG_ALL = 0, SROCM_BAG_BERNOULLI = 1 };
typedef struct srocm_bag {
    uint32_t kind;  /* SROCM_BAG_* */
    uint32_t seed;
    uint32_t round;
    uint32_t pad_;
    double fraction;
} srocm_bag;

/* LeafRange (crates/silvic-core/src/backend/mod.rs:17-22): partition[begin .. begin + count]. */
typedef struct srocm_leaf_range {
    uint32_t begin;
    uint32_t count;
} srocm_leaf_range;

/* BinSplit (crates/silvic-core/src/backend/mod.rs:24-38): rows whose bin of the feature at (group, column)
 * is set in left_bins go left. */
typedef struct srocm_bin_split {
    uint32_t group;
    uint32_t column;
    uint32_t left_bins[8];
} srocm_bin_split;

/* DeviceNode (crates/silvic-core/src/backend/mod.rs:40-46): children >= 0 are nodes, < 0 are ~leaf. */
typedef struct srocm_device_node {
    srocm_bin_split split;
    int32_t left;
    int32_t right;
} srocm_device_node;

/* Side (crates/silvic-core/src/backend/mod.rs:92-113). */
enum { SROCM_SIDE_LEFT = 0, SROCM_SIDE_RIGHT = 1 };

/* ---- device-side extension types ----------------------------------------------------------------------- */

/* SplitConfig (crates/silvic-core/src/split.rs:48-78). */
typedef struct srocm_split_config {
    int64_t min_data_in_leaf;
    double min_sum_hessian_in_leaf;
    double lambda_l1;
    double lambda_l2;
    double min_gain_to_split;
    uint64_t max_cat_to_onehot;
    uint64_t max_cat_threshold;
    double cat_l2;
    double cat_smooth;
    int64_t min_data_per_group;
} srocm_split_config;

/* LeafSums (crates/silvic-core/src/split.rs:91-97): sums in histogram units and the row count. */
typedef struct srocm_sums {
    double grad;
    double hess;
    int64_t count;
} srocm_sums;

/* SplitInfo (crates/silvic-core/src/split.rs:120-132). SplitRule::Numerical (categorical == 0): bins
 * 0..=threshold go left, the NaN bin goes left iff default_left. SplitRule::Categorical (categorical == 1): the
 * num_cat_bins bins cat_bins[0..num_cat_bins) go left, in the rule's order (split.rs:114-116); threshold and
 * default_left are 0. */
typedef struct srocm_split_info {
    int32_t found;        /* 0: the leaf has no split (Option::None) */
    int32_t feature;
    double gain;          /* best_gain - min_gain_shift */
    uint32_t threshold;
    uint32_t default_left;
    srocm_sums left;
    srocm_sums right;
    double left_output;
    double right_output;
    uint32_t categorical;
    uint32_t num_cat_bins;
    uint32_t cat_bins[256];
} srocm_split_info;

/* One tree grown on the device (Learner::grow, crates/silvic-core/src/learner.rs:121-169): LightGBM tree
 * arrays (crates/silvic-core/src/tree.rs:46-73) with thresholds as bins, plus the device splits and the
 * leaves' row ranges. Arrays are caller-allocated with room for `capacity_leaves` leaves
 * (capacity_leaves - 1 internal nodes). */
typedef struct srocm_grown_tree {
    uint32_t capacity_leaves;
    uint32_t num_leaves;          /* out */
    /* per internal node */
    int32_t *split_feature;
    uint32_t *threshold_bin;
    uint8_t *default_left;
    int32_t *left_child;
    int32_t *right_child;
    float *split_gain;            /* (gain + min_gain_to_split) as f32 */
    double *internal_value;
    double *internal_weight;
    int64_t *internal_count;
    /* per leaf */
    double *leaf_value;
    double *leaf_weight;
    int64_t *leaf_count;
    int32_t *leaf_parent;
    int32_t *leaf_depth;
    srocm_leaf_range *leaf_range;
    /* per internal node, 8 words: the bins that go left (BinSplit::left_bins; for a feature of a 2-byte group, the
     * numerical rule of srocm_group.bin_bits); a categorical node has threshold_bin 0 and default_left 0. May be
     * null. */
    uint32_t *left_bins;
} srocm_grown_tree;

/* TreeSpec (crates/silvic-core/src/learner.rs:42-54) plus the learner's own parameters. */
typedef struct srocm_grow_spec {
    srocm_split_config cfg;
    uint32_t num_leaves;
    int32_t max_depth;
    double grad_scale;            /* HistScale: real sum per histogram unit */
    double hess_scale;
    const uint8_t *feature_mask;  /* num_features; the features this tree may split on */
    srocm_leaf_range root;
    int64_t root_count;
} srocm_grow_spec;

/* ---- probes and context ---------------------------------------------------------------------------------- */

/* 1 when the HIP runtime loads and reports a gfx950 device; never aborts
 * (crates/silvic-gpu/src/cuda.rs:19-23). */
int srocm_is_available(void);

/* Opens device `ordinal` (-1: the default device). */
int srocm_create(int ordinal, void **ctx);
void srocm_destroy(void *ctx);

/* UTF-8 message of the last failure on `ctx` (or of the last srocm_create when ctx is NULL). */
const char *srocm_last_error(const void *ctx);

/* Backend::name (crates/silvic-core/src/backend/mod.rs:116-117). */
int srocm_name(void *ctx, char *buf, size_t len);

/* ---- trait Backend mirror ------------------------------------------------------------------------------- */

/* Backend::load (mod.rs:125-126): copies the training set (and validation sets, which must share its
 * layout, crates/silvic-core/src/backend/cpu.rs:707-728) into device memory. */
int srocm_load(void *ctx, const srocm_dataset *train, const srocm_dataset *const *valid, uint32_t num_valid,
               const srocm_objective *objective);

/* Backend::init_scores (mod.rs:128-129). */
int srocm_init_scores(void *ctx, uint32_t dataset, double value);

/* Backend::compute_gradients (mod.rs:131-132): f32 gradients of the training scores and their local maxima
 * (max |g|, max |h|, crates/silvic-core/src/backend/cpu.rs:757-780). */
int srocm_compute_gradients(void *ctx, double *max_abs_grad, double *max_hess);

/* Overwrites the training gradients with host-computed values (objectives whose gradients stay on the host,
 * e.g. lambdarank, crates/silvic-core/src/objective/lambdarank.rs:197); returns their maxima like
 * srocm_compute_gradients. */
int srocm_set_gradients(void *ctx, const float *grad, const float *hess, uint64_t n, double *max_abs_grad,
                        double *max_hess);

/* Reads back the training gradients and hessians the last srocm_compute_gradients / srocm_set_gradients left
 * on the device (no counterpart in the trait: for callers that check or reuse them on the host). */
int srocm_gradients(void *ctx, float *grad, float *hess, size_t len);

/* Backend::quantize (mod.rs:134-135). Units up to grad_max_q 32767 and hess_max_q 65535 (the halves of the packed
 * word), whose largest times the rows one histogram workgroup takes stays below 2^31 (SROCM_ERR_UNSUPPORTED
 * otherwise: a workgroup's sums are 32-bit). Units of more than 127 (g) or 255 (h) are an extension, accumulated in
 * separate 32-bit LDS counters rather than packed words; the slabs are laid out again when the mode changes. */
int srocm_quantize(void *ctx, const srocm_quant_spec *spec);

/* Backend::reset_partition (mod.rs:137-138). */
int srocm_reset_partition(void *ctx, const srocm_bag *bag, uint32_t *count);

/* Backend::set_histogram_features (mod.rs:140-145). */
int srocm_set_histogram_features(void *ctx, const uint8_t *used, uint32_t num_features);

/* Backend::histogram (mod.rs:147-149): `out` holds 2 * total_bins doubles, overwritten. Only quantized
 * mode runs on the device; quantized == 0 returns SROCM_ERR_UNSUPPORTED. */
int srocm_histogram(void *ctx, srocm_leaf_range leaf, int quantized, double *out, size_t len);

/* Backend::partition (mod.rs:151-152). */
int srocm_partition(void *ctx, srocm_leaf_range leaf, const srocm_bin_split *split, uint32_t *left);

/* Backend::partition_and_histogram (mod.rs:154-168), one host wait for both. */
int srocm_partition_and_histogram(void *ctx, srocm_leaf_range leaf, const srocm_bin_split *split, uint32_t side,
                                  int quantized, double *out, size_t len, uint32_t *left);

/* Backend::leaf_sums (mod.rs:170-172): out[2*i] = sum rint(g*grad_scale), out[2*i+1] = sum rint(h*hess_scale). */
int srocm_leaf_sums(void *ctx, const srocm_leaf_range *leaves, uint32_t num_leaves, float grad_scale,
                    float hess_scale, int64_t *out);

/* Backend::add_tree (mod.rs:174-175). */
int srocm_add_tree(void *ctx, const srocm_device_node *nodes, uint32_t num_nodes, const float *leaf_values,
                   uint32_t num_leaf_values);

/* Backend::scores (mod.rs:177-178). */
int srocm_scores(void *ctx, uint32_t dataset, float *out, size_t len);

/* ---- device-side extension (valid only with a local collective) ----------------------------------------- */

/* split::find_best_split (crates/silvic-core/src/split.rs:919-961) on a host histogram of `len` doubles
 * holding integer units, over `features` (their hist_offset/num_bins index `hist`), run on the device.
 * `evaluate` and `splittable` have one byte per feature. Needs no loaded dataset. Numerical, one-hot and sorted
 * categorical features (split.rs:582-844); a categorical rule's bins come back in `out->cat_bins` in the rule's
 * order. */
int srocm_find_best_split(void *ctx, const double *hist, size_t len, const srocm_feature *features,
                          uint32_t num_features, const uint8_t *evaluate, const srocm_sums *sums, double grad_scale,
                          double hess_scale, const srocm_split_config *cfg, srocm_split_info *out,
                          uint8_t *splittable);

/* Histogram slots: the learner's histograms kept on the device, for a binding that grows trees split by split over
 * the calls above (learner.rs:121-352; trees of more leaves than srocm_grow takes). They replace the host copies of
 * Learner's histograms and its subtraction (learner.rs:356-371): each slot holds 2 * total_bins int64 units in
 * srocm_histogram's order. */

/* Sets up `num_slots` slots on the loaded dataset (earlier slots and their contents are dropped). */
int srocm_hist_slots(void *ctx, uint32_t num_slots);

/* Backend::histogram (mod.rs:147-149, quantized mode) into slot `slot`; nothing comes back to the host. */
int srocm_histogram_slot(void *ctx, srocm_leaf_range leaf, uint32_t slot);

/* Backend::partition_and_histogram (mod.rs:154-168, quantized mode) with the `side` child's histogram into slot
 * `slot`; *left as srocm_partition_and_histogram returns it. */
int srocm_partition_and_histogram_slot(void *ctx, srocm_leaf_range leaf, const srocm_bin_split *split, uint32_t side,
                                       uint32_t slot, uint32_t *left);

/* learner.rs:365-367 on the device: slot `parent_slot` -= slot `child_slot`, so the parent's slot holds the other
 * child's histogram (exact integer units). */
int srocm_subtract(void *ctx, uint32_t parent_slot, uint32_t child_slot);

/* srocm_find_best_split over slot `slot` instead of a host histogram. */
int srocm_find_best_split_slot(void *ctx, uint32_t slot, const srocm_feature *features, uint32_t num_features,
                               const uint8_t *evaluate, const srocm_sums *sums, double grad_scale, double hess_scale,
                               const srocm_split_config *cfg, srocm_split_info *out, uint8_t *splittable);

/* Slot `slot` as 2 * total_bins doubles (what srocm_histogram would have returned). */
int srocm_read_slot(void *ctx, uint32_t slot, double *out, size_t len);

/* Learner::grow (crates/silvic-core/src/learner.rs:121-169) with every histogram, subtraction, split search
 * and partition on the device and one readback of the finished tree. Quantized mode only. */
int srocm_grow(void *ctx, const srocm_grow_spec *spec, srocm_grown_tree *out);


/* Training parameters of the boosting loop (crates/silvic-core/src/config.rs:123-167 defaults; the fields
 * boosting.rs/learner.rs/split.rs read). */
typedef struct srocm_train_params {
    uint32_t objective;            /* SROCM_OBJ_REGRESSION / SROCM_OBJ_BINARY */
    uint32_t num_leaves;
    double sigmoid;
    double learning_rate;
    int32_t max_depth;
    uint32_t num_grad_quant_bins;  /* even, 2..=64 as the reference (config.rs:416-421); up to 32766 as an
                                    * extension (g_q within +-16383, h_q at most 32766: 16-bit units) */
    srocm_split_config cfg;
    double bagging_fraction;
    uint32_t bagging_freq;
    uint32_t bagging_seed;
    double feature_fraction;
    uint32_t feature_fraction_seed;
    uint32_t data_random_seed;
    uint8_t stochastic_rounding;
    uint8_t quant_train_renew_leaf;
    uint8_t boost_from_average;
    uint8_t pad_;
} srocm_train_params;

/* train_from's set-up after `load` (crates/silvic-core/src/boosting.rs:100-108): the initial score
 * (BoostFromAverage) written into every dataset's scores. */
int srocm_boost_init(void *ctx, const srocm_train_params *params, double *init_score);

/* `count` boosting iterations from `first_iteration` (Trainer::train_one_iter, boosting.rs:227-324): device
 * gradients, quantization, partition reset, whole-tree growth on the device, leaf renewal, shrinkage and
 * the score update. trees[i] receives iteration i's tree as the model stores it (shrunk; the first tree
 * with the initial score folded in). `*trained` is the number of trees added; it is below `count` when a
 * tree could not split (training ends, boosting.rs:275-278); a first tree that cannot split becomes the
 * constant tree holding the initial score. */
int srocm_boost(void *ctx, const srocm_train_params *params, uint32_t first_iteration, uint32_t count,
                srocm_grown_tree *trees, uint32_t *trained);

/* Reads back the first `len` row ids of the backend's partition (the order srocm_reset_partition,
 * srocm_partition and srocm_grow left them in; a grown tree's leaves hold their rows' ranges). No counterpart in
 * the trait: for callers that check or reuse the row order on the host. `len` is at most the training rows. */
int srocm_partition_rows(void *ctx, uint32_t *out, size_t len);

/* The quantized histogram of a leaf's rows into a caller-owned DEVICE buffer `out` of `len` = 2 * total_bins
 * int64 values (the {g, h} sums of quantized units per bin, in the flat histogram order srocm_histogram uses),
 * allocating nothing: no hipMalloc, no hipFree, no allocating library call. It has no counterpart in the
 * reference; it is for callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation). The per-workgroup partials go to a
 * 16 MiB scratch array that each GPU holds until the process ends and that every call on that GPU shares, so
 * calls that overlap on one GPU race. At most 16 MiB / (256 * slab width * 8 B) workgroups run (64 for 128-wide
 * slabs); a leaf whose rows per workgroup times the largest quantized unit could pass 2^31 is refused with
 * SROCM_ERR_UNSUPPORTED. Runs on the context's stream; waits for the result when `wait` is nonzero. */
int srocm_histogram_noalloc(void *ctx, srocm_leaf_range leaf, int64_t *out, size_t len, int wait);

/* Per-kernel timing with HIP events on the backend's stream, and algorithmic byte counts; no counterpart in the
 * reference (a measurement hook). srocm_profile: enable (1), enable with the line model (2: after every split
 * step's k_step_rows launches, kernels that count the memory lines its gathers touch, values [15]-[24]), or disable (0);
 * each resets the counters.
 * srocm_profile_read writes min(len, SROCM_PROFILE_VALUES) values:
 *   [0] k_hist launches (root and trait histograms, one per slab)   [1] their ms   [2] their algorithmic bytes
 *   [3] k_step_rows launches (split steps: partition + built-child histogram)   [4] their ms
 *   [5] their algorithmic bytes (9 B per partitioned row + used columns + 4 B per histogrammed row)
 *   [6] histogram builds   [7] rows histogrammed   [8] rows x used columns   [9] rows partitioned
 *   [10] trait partition launches   [11] their ms (count + scatter + copy back)
 *   [12] device-growth split steps   [13] leaves they expanded   [14] of those, splits the trees kept
 *   line model (mode 2; split steps, the first slab): [15] parent rows partitioned   [16] distinct 128-byte lines
 *   of the column-major split-feature bins they lie in, per job   [17] built-child rows histogrammed   [18] distinct
 *   lines of the packed gradients they lie in   [19] split-bin lines counted once per step over every job splitting
 *   on the same feature   [20] partials written   [21] of those, packed (256 x slab width x 4 bytes; the others
 *   {g, h} pairs, twice that)   [22]-[24] the sparse jobs' (fewer than two parent rows a split-bin line) parent rows,
 *   split-bin lines and built rows
 *   [25] lambdarank gradient computations whose device-made normalization factors were flagged (some row's f32
 *   gradient could depend on the last bit of the C library's log2) and made again with the host's (counted in every
 *   mode; normally 0)
 * Algorithmic bytes of a k_hist build: rows x (the used features' bin bytes, two for a two-byte bin, + 4 B gradients
 * + 4 B row id) + 2 x 4 B x the used features' bins (the output).
 * Builds whose row count only the device knows (partition_and_histogram) add launches and time but no rows. */
#define SROCM_PROFILE_VALUES 26
int srocm_profile(void *ctx, int enable);
int srocm_profile_read(void *ctx, double *out, uint32_t len);

/* The loaded training set's slab layout (no counterpart in the reference: the layout is this backend's), for
 * measurement and inspection. Writes 4 values per slab, for up to `cap` slabs: LDS columns, row bytes, features a
 * column (0: stacked by bin count), flags (1: two-byte bins, 2: separate 32-bit g and h counters, 4: stacked), and
 * the slab count into *count. */
int srocm_slab_layout(void *ctx, uint32_t *out, uint32_t cap, uint32_t *count);

#ifdef __cplusplus
}
#endif

#endif /* SILVIC_ROCM_H */
