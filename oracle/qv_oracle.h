/*
 * qv_oracle.h -- CPU restatement of the Quiver query path (TEST INFRASTRUCTURE).
 *
 * This library is the test oracle of the HIP path: only tests/, the smoke test and
 * bench.py's cpu_baseline leg may load it.  The product never links it.
 *
 * Every function restates a reference routine; the file:line it follows is in
 * the comment above its definition in qv_oracle.c (paths are relative to the
 * ruc-system/quiver-ae checkout).
 *
 * Pinning status of each function (what fixes its output besides this code):
 *   qvo_lut_build      closed form sum_{i in chunk}(fl(q_i-mu_i)-P[c][i])^2,
 *                      float64 bound + zero-at-pivot invariant (tests/test_oracle.py)
 *   qvo_adc            closed form sum_m LUT[m][code_m]; float64 bound and
 *                      bit-exact sequential order (tests/test_oracle.py)
 *   qvo_exact_l2       integer brute force for uint8/int8 (bit-exact), float64
 *                      bound for float (tests/test_oracle.py)
 *   qvo_search_one     complete-graph known answer (ef >= n -> brute-force top-k
 *                      plus the entry-duplicate quirk), hand graphs checked step
 *                      by step, gpruning/none invariants (tests/test_oracle_search.py)
 *   qvo_recall         the reference's own known-answer test
 *                      (bin/common/search_setup_test.cpp:67-81) and the reference
 *                      header compiled into oracle/_ref when it is present
 *   qvo_adc_topk       brute force sort by (dist, sequence) (tests/test_oracle.py)
 *   qvo_nav_entry      complete nav graph known answer (exact nearest nav node),
 *                      chain graphs (greedy descent stops at the reachable local
 *                      minimum), a hand-traced 2- and 3-node graph where the
 *                      empty-slot swap fires, the per-chunk break traced on a
 *                      graph with a short row (tests/test_oracle_nav.py).  One case
 *                      stays unpinned: three or more copies of one id in the
 *                      queue with differing visited bits, where the reference's
 *                      same-address shared-memory stores race; this restatement
 *                      ORs all of them.
 */
#ifndef QV_ORACLE_H
#define QV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { QVO_UINT8 = 0, QVO_FLOAT = 1, QVO_INT8 = 2 };
enum { QVO_EXIT_NONE = 0, QVO_EXIT_GPRUNING = 2 };
enum { QVO_OK = 0, QVO_EINVAL = -1, QVO_EMERGE = -2 };

#define QVO_PAGE_SIZE 4096
#define QVO_NUM_PIVOTS 256

/* View of one DiskANN-format index held in host memory (heap backend). */
typedef struct {
  int dtype;               /* QVO_UINT8 / QVO_FLOAT / QVO_INT8 */
  int dim;                 /* vector dimension d */
  int64_t num_points;      /* n */
  int max_m;               /* R, slots per adjacency record */
  int64_t medoid;          /* entry point */
  int64_t node_size;       /* bytes per node record */
  int64_t nodes_per_page;  /* records per 4 KB page */
  int64_t data_size;       /* d * sizeof(element) */
  const uint8_t* pages;    /* page image without the header page */
  int num_chunks;          /* M */
  const uint8_t* codes;    /* [n][M] PQ codes */
  const float* centroid;   /* [d] */
  const float* pivots_t;   /* [d][256] transposed pivots */
  const int32_t* chunk_id; /* [d] chunk of each dimension */
} qvo_index;

/* Navigation graph (the reference's NavGraph, src/shared/index/nav_graph.cu):
 * a small graph over sampled base vectors whose greedy search picks each
 * query's entry node. */
typedef struct {
  int dtype;               /* same element type as the base index */
  int dim;
  int64_t num_node;
  int max_m;               /* row stride of graph, 1..32 */
  int start;               /* root of the nav search */
  const void* data;        /* [num_node][dim] elements */
  const int32_t* graph;    /* [num_node][max_m], -1 after each node's degree */
  const int32_t* mapping;  /* [num_node] nav id -> base id */
} qvo_nav;

typedef struct {
  int topk;
  int ef_search;
  int pipe_width;          /* W >= 1; lanes are served instantly (HBM-resident) */
  int early_exit;          /* QVO_EXIT_NONE or QVO_EXIT_GPRUNING */
  int gpruning_warmup;     /* reference CLI default 10 */
  int gpruning_patience;   /* reference CLI default 8 */
  const qvo_nav* nav;      /* entry from the nav search when not NULL, else the medoid */
  /* per-step recall (kernel_q1.cuh:354-364, 662-667; search.cu:100-102): when
   * sr_gt is not NULL, query i checks after each step how many of its top-k
   * ids appear in ground-truth row i % sr_count (sr_width ids) and stops once
   * that count reaches sr_required; sr_step[i] receives that step (-1 when
   * never reached) and sr_hits[i] the count then (else the final count).
   * Pipe width 1 only (search.cu:493-496).  sr_step/sr_hits are used by the
   * batch calls (qvo_search, qvo_search_timed), indexed by query. */
  const int32_t* sr_gt;
  int sr_width;
  int sr_count;
  int sr_required;
  int32_t* sr_step;
  int32_t* sr_hits;
} qvo_search_params;

/* Entry node of raw query q from the nav graph (base id).  `fallback` is
 * returned when the queue's slot 0 ends empty (the reference reads past
 * nav_mapping there). */
int64_t qvo_nav_entry(const qvo_nav* nav, const float* q, int64_t fallback);

/* LUT build.  lut is [M][256]; q_used receives fl(fl(q-mu)+mu), the query the
 * reference's exact-distance stage sees after init_query restores it. */
void qvo_lut_build(const qvo_index* ix, const float* q, float* lut, float* q_used);

/* Raw variant for microbenchmarks: explicit tables instead of an index. */
void qvo_lut_build_raw(int dim, int num_chunks, const float* centroid,
                       const float* pivots_t, const int32_t* chunk_id,
                       const float* q, float* lut, float* q_used);

/* Sequential fp32 ADC of one code row. */
float qvo_adc(const float* lut, int num_chunks, const uint8_t* code_row);

/* Exact squared L2 in the reference's lane order (32 strided partial sums,
 * fused multiply-add, then a shuffle-down tree). x points at dtype elements. */
float qvo_exact_l2(const float* q, const void* x, int dtype, int dim);

/* Full deterministic beam search of one query.  Outputs topk ids (-1 padded),
 * distances (+inf padded), the found count and the number of expanded hops.
 * Returns QVO_OK, QVO_EINVAL, or QVO_EMERGE if the merge path met duplicate
 * keys inside one adjacency list (outside the reference's domain). */
int qvo_search_one(const qvo_index* ix, const float* q, const qvo_search_params* p,
                   int32_t* ids, float* dists, int32_t* found, int32_t* hops);
/* qvo_search_one that also writes the node expanded at each step (trace[s] for
 * step s + 1, the first trace_cap steps; the entry is step 1). */
int qvo_search_trace(const qvo_index* ix, const float* q, const qvo_search_params* p,
                     int32_t* ids, float* dists, int32_t* found, int32_t* hops,
                     int32_t* trace, int trace_cap);

/* All queries, OpenMP over queries with `threads` threads (<=0: all cores).
 * Returns the first non-OK status, else QVO_OK. */
int qvo_search(const qvo_index* ix, const float* queries, int64_t nq,
               const qvo_search_params* p, int threads, int32_t* ids,
               float* dists, int32_t* found, int32_t* hops);
/* qvo_search that also writes each query's wall time in seconds (for the CPU
 * baseline's per-query latency; seconds may be NULL). */
int qvo_search_timed(const qvo_index* ix, const float* queries, int64_t nq,
                     const qvo_search_params* p, int threads, int32_t* ids,
                     float* dists, int32_t* found, int32_t* hops, double* seconds);

/* Recall@k as the reference computes it: hits of results[i][0..k) in the set
 * gt[i][0..k), divided by n*k. */
double qvo_recall(const int32_t* results, const int32_t* gt, int64_t nq,
                  int gt_width, int k);

/* ADC + top-k microbenchmark semantics for one query: distances of
 * codes[ids[s]] for s in [0, nids), the k smallest under (dist, s) order.
 * Returns the ids and distances of the winners and the sum of all distances
 * (double) through *dist_sum when it is not NULL. */
void qvo_adc_topk(const float* lut, int num_chunks, const uint8_t* codes,
                  const int32_t* ids, int64_t nids, int k, int32_t* out_ids,
                  float* out_dists, double* dist_sum);

/* Brute-force exact ground truth (float64 accumulation, ties by id) used to
 * measure recall of small test indexes. base is [n][d] of dtype. */
void qvo_ground_truth(const void* base, int dtype, int64_t n, int dim,
                      const float* queries, int64_t nq, int k, int threads,
                      int32_t* gt_ids, float* gt_dists);

#ifdef __cplusplus
}
#endif
#endif
