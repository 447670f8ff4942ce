/*
 * hist_oracle.h -- CPU restatement of the reference's histogram tree-boosting
 * path (tree_method='hist', depthwise growth).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker: it may be
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg, and by nothing else.  The product library never links or calls it.
 *
 * Every function follows a reference file:line (paths relative to the
 * reference repository root); see the comments in hist_oracle.c.
 */
#ifndef HIST_ORACLE_H
#define HIST_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Objectives (same codes as the reference: src/learner.cpp objective map). */
enum { ORACLE_OBJ_SQUARED_ERROR = 0, ORACLE_OBJ_LOGISTIC = 1, ORACLE_OBJ_LOGITRAW = 2 };

typedef struct {
  int32_t objective;
  int32_t max_depth;
  int32_t max_bin;
  int32_t fma_contract;      /* 1: binary64 gain uses fused multiply-adds (arm64 CPU build) */
  float eta;
  float reg_lambda;
  float reg_alpha;
  float min_child_weight;
  float max_delta_step;
  float min_split_loss;
  float scale_pos_weight;
  float base_score;          /* used when has_base_score != 0 */
  int32_t has_base_score;
  int32_t nthread;           /* histogram threads; results never depend on it */
  float subsample;           /* uniform row sampling when < 1 (src/sampling.cpp:11-74) */
  float colsample_bytree;    /* per-tree feature sampling when < 1 (src/tree.cpp:28-45) */
  uint32_t seed;             /* "seed" parameter; 0 keeps the engine's default state */
  const int32_t* monotone;   /* per feature -1, 0 or 1 (monotone_constraints); NULL: none */
  int32_t std_shuffle;       /* column sample's std::shuffle: 0 libstdc++ (x86-64), 1 libc++ (macOS) */
  int32_t seed_per_iteration; /* reseed the engine with seed * 127 + round before each round */
} OracleParams;

/* One tree node; field meanings follow the reference's Node plus base_weights
 * (include/metalgb/shared.h:27-31, src/tree.cpp:1049-1104). */
typedef struct {
  int32_t left, right, parent, feature;
  float threshold, leaf, cover, gain;
  uint32_t default_left;
  float base_weight;
} OracleNode;

/* Best split candidate of one (node, feature) or one node; mirrors the
 * reference's Split (include/metalgb/shared.h:124-134) restricted to the
 * scalar numeric path. */
typedef struct {
  float gain, threshold, left_weight, right_weight, left_h, right_h;
  float parent_weight, total_g, total_h;
  int32_t feature;
  uint32_t default_left;
  uint32_t bin;              /* candidate bin b of the chosen split */
  int64_t left_g, left_hs, right_g, right_hs;
} OracleSplit;

/* --- quantile sketch and bins ------------------------------------------ */
uint32_t oracle_sketch_budget(uint32_t bins, uint32_t count);
/* cuts: cols*max_bin floats; counts: cols; minima: cols.  weights may be NULL. */
int oracle_sketch_cuts(const float* X, uint32_t rows, uint32_t cols, const float* weights,
                       uint32_t max_bin, float* cuts, uint32_t* counts, float* minima);
/* Test hook: ids 0..n-1 of elements with these keys in the order the
 * sketch's std::sort restatement (libstdc++'s steps) leaves them; returns the
 * number of heap-sort fallbacks it took. */
uint64_t oracle_std_sort_order(const uint32_t* keys, uint32_t n, uint32_t* order);
/* Row-major bins[r*cols+f]; 0xFFFF marks missing. */
void oracle_quantize(const float* X, uint32_t rows, uint32_t cols, const float* cuts,
                     const uint32_t* counts, uint32_t max_bin, uint16_t* bins);

/* --- gradients ----------------------------------------------------------- */
float oracle_base_score(int32_t objective, const float* labels, const float* weights, uint32_t rows,
                        float scale_pos_weight);
float oracle_base_margin(int32_t objective, float base_score);
float oracle_sigmoid(float x);
void oracle_sigmoid_array(const float* in, float* out, uint64_t count);
void oracle_gradients(int32_t objective, const float* margin, const float* labels, const float* weights,
                      uint32_t rows, float scale_pos_weight, float* grad, float* hess);
/* Power-of-two fixed-point scale of one gradient column. */
float oracle_gradient_scale(const float* values, uint32_t rows);
void oracle_quantize_gradients(const float* grad, const float* hess, uint32_t rows, float scale_g,
                               float scale_h, int64_t* qg, int64_t* qh);

/* --- histograms and splits ---------------------------------------------- */
/* hist: cols*(max_bin+1)*2 int64 (g, h) per bin, bin max_bin = missing. */
void oracle_histogram(const uint16_t* bins, uint32_t cols, uint32_t max_bin, const uint32_t* rows,
                      uint32_t count, const int64_t* qg, const int64_t* qh, int64_t* hist);
/* Evaluate one feature of one node; total_g/total_h are the node's integer sums. */
void oracle_evaluate_feature(const int64_t* feature_hist, uint32_t count, const float* cuts, float minimum,
                             int64_t total_g, int64_t total_h, float scale_g, float scale_h,
                             const OracleParams* p, int32_t feature, OracleSplit* out);
float oracle_weight(double G, double H, const OracleParams* p);
float oracle_gain(double G, double H, float w, const OracleParams* p);

/* --- sampling ------------------------------------------------------------ */
/* MT19937 (Matsumoto and Nishimura 1998), the engine behind std::mt19937. */
typedef struct { uint32_t state[624]; uint32_t next; } OracleMT;
void oracle_mt_seed(OracleMT* g, uint32_t seed);
uint32_t oracle_mt_next(OracleMT* g);
/* Uniform row sampling: 1 if row `row` is kept in a round whose seed is `seed`
 * (kernels/sampling.metal.h:1-30). */
int oracle_sample_row(uint32_t seed, uint32_t row, float subsample);
/* std::shuffle(v, v + n, g) with the draws of libstdc++ (model 0) or libc++
 * (model 1). */
void oracle_std_shuffle(uint32_t* v, uint32_t n, OracleMT* g, int32_t model);
/* Per-tree feature sample of n features: writes the sorted subset to out and
 * returns its size (src/tree.cpp:28-45, std::shuffle of the given model). */
uint32_t oracle_sample_columns(uint32_t n, float fraction, uint32_t seed, int32_t model, uint32_t* out);

/* --- training ------------------------------------------------------------ */
uint32_t oracle_max_nodes(int32_t max_depth);
/* Trains `rounds` trees.  trees: rounds*oracle_max_nodes(max_depth) nodes;
 * tree_sizes: rounds; margin: rows (training margin after the last round).
 * custom_grad/custom_hess (optional, rounds*rows) replace the objective. */
int oracle_train(const float* X, uint32_t rows, uint32_t cols, const float* labels, const float* weights,
                 const OracleParams* p, uint32_t rounds, const float* custom_grad, const float* custom_hess,
                 OracleNode* trees, uint32_t* tree_sizes, float* margin, float* base_score_out,
                 float* cuts_out, uint32_t* cut_counts_out);
/* Margin of new rows: base_margin + sum of tree leaves (float traversal). */
void oracle_predict_margin(const float* X, uint32_t rows, uint32_t cols, const OracleNode* trees,
                           const uint32_t* tree_sizes, uint32_t rounds, uint32_t stride, float base_margin,
                           float* out);

/* Evaluation metrics (src/metrics.cpp:8-159).  kind numbers follow the
 * reference's metric table: 0 rmse, 1 mae, 2 rmsle, 3 logloss, 6 error,
 * 7 mape, 8 mphe, 9 poisson-nloglik, 10 gamma-deviance, 11 tweedie-nloglik,
 * 12 gamma-nloglik.  out = (sum of weight * loss, sum of weight) in the
 * reference's fp32 order (kernels/boost.metal:2225-2295). */
void oracle_metric_sum(const float* pred, const float* labels, const float* weights, uint32_t rows, uint32_t kind,
                       float parameter, float out[2]);
/* ROC-AUC (pr = 0) or PR-AUC (pr = 1) area, positive and negative weight in
 * binary64 (kernels/radix_sort.metal.h:427-790). */
void oracle_metric_auc(const float* pred, const float* labels, const float* weights, uint32_t rows, int pr,
                       double out[3]);
/* Fold of each row for xgboost.cv (src/c_api.cpp:1018-1110); model selects
 * std::shuffle's draws as in oracle_std_shuffle. */
void oracle_cv_folds(uint32_t rows, int nfold, uint32_t seed, int shuffle, int stratified, const float* labels,
                     int32_t model, int32_t* fold);

#ifdef __cplusplus
}
#endif
#endif
