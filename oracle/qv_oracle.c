/*
 * qv_oracle.c -- CPU restatement of the Quiver query path (TEST INFRASTRUCTURE).
 *
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, always as the test oracle.  Citations are ruc-system/quiver-ae paths.
 *
 * Floating point: every `a += b * b` of the reference is written as fmaf(b, b, a)
 * because nvcc contracts that statement to one FFMA under its default
 * --fmad=true; the bits of the reference binary itself cannot be observed here,
 * so this contraction is the one unpinnable assumption of the restatement.
 */
#define _POSIX_C_SOURCE 199309L /* clock_gettime under -std=c11 */
#include "qv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <time.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ID_MASK 0x7fffffffu
#define VISITED 0x80000000u

/* ------------------------------------------------------------------------ */
/* LUT build: src/shared/index/pq_device.cuh:9-36 (and the slot-indexed copy  */
/* at src/quiver/kernel_core/kernel_qi.cuh:348-372).                          */
/* q' = fl(q - mu) in place; for i = 0..d-1 in order, for every pivot j:     */
/*   LUT[chunk_id[i]][j] += (q'_i - P^T[i][j])^2 ; then q = fl(q' + mu).     */
/* ------------------------------------------------------------------------ */
void qvo_lut_build_raw(int dim, int num_chunks, const float* centroid,
                       const float* pivots_t, const int32_t* chunk_id,
                       const float* q, float* lut, float* q_used) {
  float* qc = (float*)malloc(sizeof(float) * (size_t)dim);
  memset(lut, 0, sizeof(float) * (size_t)num_chunks * QVO_NUM_PIVOTS);
  for (int i = 0; i < dim; i++) qc[i] = q[i] - centroid[i];
  for (int i = 0; i < dim; i++) {
    float* row = lut + (size_t)chunk_id[i] * QVO_NUM_PIVOTS;
    const float* pt = pivots_t + (size_t)i * QVO_NUM_PIVOTS;
    for (int j = 0; j < QVO_NUM_PIVOTS; j++) {
      float diff = qc[i] - pt[j];
      row[j] = fmaf(diff, diff, row[j]);
    }
  }
  if (q_used) {
    for (int i = 0; i < dim; i++) q_used[i] = qc[i] + centroid[i];
  }
  free(qc);
}

void qvo_lut_build(const qvo_index* ix, const float* q, float* lut, float* q_used) {
  qvo_lut_build_raw(ix->dim, ix->num_chunks, ix->centroid, ix->pivots_t,
                    ix->chunk_id, q, lut, q_used);
}

/* ------------------------------------------------------------------------ */
/* ADC: src/quiver/kernel_core/kernel_helpers.cuh:280-285.                    */
/* dist = 0; for j = 0..M-1: dist += LUT[j*256 + code[j]]  (fp32, in order)  */
/* ------------------------------------------------------------------------ */
float qvo_adc(const float* lut, int num_chunks, const uint8_t* code_row) {
  float dist = 0.0f;
  for (int j = 0; j < num_chunks; j++)
    dist += lut[(size_t)j * QVO_NUM_PIVOTS + code_row[j]];
  return dist;
}

/* ------------------------------------------------------------------------ */
/* Exact distance: src/shared/common/gpu_primitives.cuh:26-44                 */
/* (square_sum_32): lane l of 32 accumulates i = l, l+32, ... with           */
/* val += diff*diff, then val += shfl_down(val, off) for off = 16..1; lane 0 */
/* holds the result.                                                          */
/* ------------------------------------------------------------------------ */
static inline float elem_as_float(const void* x, int dtype, int i) {
  if (dtype == QVO_FLOAT) return ((const float*)x)[i];
  if (dtype == QVO_INT8) return (float)((const int8_t*)x)[i];
  return (float)((const uint8_t*)x)[i];
}

float qvo_exact_l2(const float* q, const void* x, int dtype, int dim) {
  float v[32];
  for (int lane = 0; lane < 32; lane++) {
    float val = 0.0f;
    for (int i = lane; i < dim; i += 32) {
      float diff = q[i] - elem_as_float(x, dtype, i);
      val = fmaf(diff, diff, val);
    }
    v[lane] = val;
  }
  for (int off = 16; off > 0; off /= 2) {
    float nv[32];
    for (int lane = 0; lane < 32; lane++)
      nv[lane] = v[lane] + ((lane + off < 32) ? v[lane + off] : v[lane]);
    memcpy(v, nv, sizeof(v));
  }
  return v[0];
}

/* ------------------------------------------------------------------------ */
/* lower_bound: src/shared/common/gpu_primitives.cuh:140-153.                 */
/* First index in [l, r) whose (dist, id&mask) is not less than (d, x&mask). */
/* ------------------------------------------------------------------------ */
static int ref_lower_bound(const float* dist_arr, const uint32_t* id_arr, int l,
                           int r, float d, uint32_t x) {
  x &= ID_MASK;
  while (l < r) {
    int mid = (l + r) / 2;
    if (dist_arr[mid] < d ||
        (dist_arr[mid] == d && (id_arr[mid] & ID_MASK) < x)) {
      l = mid + 1;
    } else {
      r = mid;
    }
  }
  return l;
}

/* Per-query search state: the reference keeps these per task slot in global */
/* memory (src/quiver/search.cu:474-480) and in shared scratch               */
/* (src/quiver/kernel_core/kernel_q1.cuh:32-40).                             */
typedef struct {
  int ef, max_m, topk;
  uint32_t* nid;   /* beam ids, capacity ef + max_m */
  float* ndist;    /* beam PQ distances */
  int ctx_size;    /* Data::size */
  int32_t* nns;    /* top-k ids */
  float* tdist;    /* top-k exact distances */
  int fc;          /* found count */
  /* merge scratch (tmp_*, mv_*) */
  uint32_t* tmp_id;
  float* tmp_dist;
  uint32_t* mv_id;
  float* mv_dist;
  int* mv_pos;
  unsigned char* written;
} qstate;

static const uint8_t* node_record(const qvo_index* ix, int64_t node) {
  int64_t page = node / ix->nodes_per_page;
  int64_t off = (node % ix->nodes_per_page) * ix->node_size;
  return ix->pages + page * QVO_PAGE_SIZE + off;
}

/* ------------------------------------------------------------------------ */
/* persistent_merge_data: src/quiver/kernel_core/kernel_helpers.cuh:232-357.  */
/*  - sz = min(ctx.size, ef) (:253-255), tmp[0,sz) = beam (:265-268)           */
/*  - tmp[sz+t] = (nbr_t, ADC(nbr_t)) for t < deg (:271-286)                  */
/*  - merge-path sort of the deg new pairs, rounds len = 2,4,.. < 2*deg        */
/*    (:300-329)                                                              */
/*  - merge into the beam; a new id equal to the old one at its lower bound    */
/*    goes right after it (:331-348)                                         */
/*  - keep min(sz+deg, 2*ef) entries (:350-355)                               */
/* The reference assumes every key of a round lands on a distinct slot; two    */
/* equal keys inside one adjacency list break that and are reported.          */
/* ------------------------------------------------------------------------ */
static int merge_data(const qvo_index* ix, qstate* s, const float* lut, int64_t node) {
  const uint8_t* rec = node_record(ix, node);
  const uint32_t* nbrs = (const uint32_t*)(rec + ix->data_size);
  int sz = s->ctx_size < s->ef ? s->ctx_size : s->ef;
  int deg = (int)nbrs[0];
  for (int i = 0; i < sz; i++) {
    s->tmp_id[i] = s->nid[i];
    s->tmp_dist[i] = s->ndist[i];
  }
  for (int t = 0; t < deg; t++) {
    uint32_t v = nbrs[t + 1];
    s->tmp_id[sz + t] = v;
    s->tmp_dist[sz + t] =
        qvo_adc(lut, ix->num_chunks, ix->codes + (int64_t)v * ix->num_chunks);
  }
  uint32_t* tid_ = s->tmp_id + sz;
  float* tdi_ = s->tmp_dist + sz;
  for (int len = 2; len < 2 * deg; len *= 2) {
    for (int t = 0; t < deg; t++) {
      int start = (t / len) * len;
      int mid = start + len / 2 < deg ? start + len / 2 : deg;
      int end = start + len < deg ? start + len : deg;
      if (t >= start && t < mid) {
        int id = ref_lower_bound(tdi_ + mid, tid_ + mid, 0, end - mid, tdi_[t], tid_[t]);
        s->mv_pos[t] = id + t;
      }
      if (t >= mid && t < end) {
        int id = ref_lower_bound(tdi_, tid_, start, mid, tdi_[t], tid_[t]);
        s->mv_pos[t] = id + t - mid;
      }
    }
    memset(s->written, 0, (size_t)deg);
    for (int t = 0; t < deg; t++) {
      int p = s->mv_pos[t];
      if (s->written[p]) return QVO_EMERGE;
      s->written[p] = 1;
      s->mv_id[p] = tid_[t];
      s->mv_dist[p] = tdi_[t];
    }
    for (int t = 0; t < deg; t++) {
      tid_[t] = s->mv_id[t];
      tdi_[t] = s->mv_dist[t];
    }
  }
  for (int t = 0; t < deg; t++) {
    int id = ref_lower_bound(s->tmp_dist, s->tmp_id, 0, sz, tdi_[t], tid_[t]);
    if (id != sz && ((s->tmp_id[id] ^ tid_[t]) & ID_MASK) == 0) id++;
    s->mv_pos[sz + t] = id + t;
  }
  for (int i = 0; i < sz; i++) {
    int id = ref_lower_bound(tdi_, tid_, 0, deg, s->tmp_dist[i], s->tmp_id[i]);
    s->mv_pos[i] = id + i;
  }
  memset(s->written, 0, (size_t)(sz + deg));
  for (int i = 0; i < sz + deg; i++) {
    int p = s->mv_pos[i];
    if (s->written[p]) return QVO_EMERGE;
    s->written[p] = 1;
    s->mv_id[p] = s->tmp_id[i];
    s->mv_dist[p] = s->tmp_dist[i];
  }
  int target = sz + deg < 2 * s->ef ? sz + deg : 2 * s->ef;
  for (int i = 0; i < target; i++) {
    s->nid[i] = s->mv_id[i];
    s->ndist[i] = s->mv_dist[i];
  }
  s->ctx_size = target;
  return QVO_OK;
}

/* ------------------------------------------------------------------------ */
/* Top-k insert: retset_push_topk_le32 (kernel_helpers.cuh:65-104) and        */
/* retset_push_32 (gpu_primitives.cuh:99-138) share one semantics: insert    */
/* after every element <= value, capacity k, size grows to at most k.        */
/* Called only when fc < k or value < D[k-1] (kernel_helpers.cuh:478-479).   */
/* ------------------------------------------------------------------------ */
static void topk_push(qstate* s, float value, int32_t id) {
  int k = s->topk;
  int pos = 0;
  while (pos < s->fc && s->tdist[pos] <= value) pos++;
  int new_size = s->fc < k ? s->fc + 1 : k;
  for (int i = new_size - 1; i > pos; i--) {
    s->tdist[i] = s->tdist[i - 1];
    s->nns[i] = s->nns[i - 1];
  }
  if (pos < new_size) {
    s->tdist[pos] = value;
    s->nns[pos] = id;
  }
  s->fc = new_size;
}

/* ------------------------------------------------------------------------ */
/* persistent_visit_select_dualwarp: kernel_helpers.cuh:422-489.              */
/* warp 0: drop entries whose masked id equals the previous entry's          */
/*   (:440-455), pick the first unvisited index; take it only if < ef         */
/*   (:456-470), size = min(sz, ef) (:471).                                   */
/* warp 1: exact distance of the expanded node and top-k insert (:475-485).  */
/* ------------------------------------------------------------------------ */
static int32_t visit_select(const qvo_index* ix, qstate* s, const float* q_used,
                            int64_t node) {
  int32_t next = -1;
  int sz = s->ctx_size;
  if (sz != 0) {
    int w = 0;
    /* flags are taken on the uncompacted array (see the chunked loop at     */
    /* :442-454: a slot below i is only rewritten after it has been read).   */
    uint32_t prev = 0;
    for (int i = 0; i < sz; i++) {
      uint32_t cur = s->nid[i];
      float cd = s->ndist[i];
      int dup = (i != 0) && (((cur ^ prev) & ID_MASK) == 0);
      prev = cur;
      if (!dup) {
        s->nid[w] = cur;
        s->ndist[w] = cd;
        w++;
      }
    }
    sz = w;
    int id = sz + 1;
    for (int i = 0; i < sz; i++) {
      if ((s->nid[i] & VISITED) == 0) { id = i; break; }
    }
    if (id < s->ef && id < sz) {
      next = (int32_t)(s->nid[id] & ID_MASK);
      s->nid[id] |= VISITED;
    }
    s->ctx_size = sz < s->ef ? sz : s->ef;
  }
  if (node != -1) {
    const uint8_t* rec = node_record(ix, node);
    float dist = qvo_exact_l2(q_used, rec, ix->dtype, ix->dim);
    if (s->fc < s->topk || dist < s->tdist[s->topk - 1])
      topk_push(s, dist, (int32_t)node);
  }
  return next;
}

/* persistent_select_next_no_compact: kernel_helpers.cuh:491-518. */
static int32_t select_next_no_compact(qstate* s) {
  int sz = s->ctx_size < s->ef ? s->ctx_size : s->ef;
  if (sz == 0) return -1;
  int id = sz + 1;
  for (int i = 0; i < sz; i++) {
    if ((s->nid[i] & VISITED) == 0) { id = i; break; }
  }
  int32_t next = -1;
  if (id < sz) {
    next = (int32_t)(s->nid[id] & ID_MASK);
    s->nid[id] |= VISITED;
  }
  s->ctx_size = sz;
  return next;
}

/* gpruning bookkeeping: kernel_q1.cuh:294-315 (boot) and :524-545 (pipe). */
typedef struct {
  int no_improve, last_fc;
  float last_top1, last_topk;
} gprune;

static int gpruning_step(const qvo_search_params* p, const qstate* s, gprune* g,
                         int step) {
  int k = s->topk;
  int improved = s->fc > g->last_fc || s->tdist[0] < g->last_top1 ||
                 s->tdist[k - 1] < g->last_topk;
  if (step < p->gpruning_warmup) {
    g->no_improve = 0;
  } else {
    g->no_improve = improved ? 0 : g->no_improve + 1;
  }
  g->last_fc = s->fc;
  g->last_top1 = s->tdist[0];
  g->last_topk = s->tdist[k - 1];
  return p->early_exit == QVO_EXIT_GPRUNING && step >= p->gpruning_warmup &&
         p->gpruning_patience > 0 && g->no_improve >= p->gpruning_patience;
}

/* ------------------------------------------------------------------------ */
/* Nav entry: inkernel_nav_entry, src/quiver/kernel_core/inkernel_nav.cuh:    */
/* 61-200, as the persistent kernel launches it (128 threads = 4 warps,       */
/* search.cu:903).  A 32-slot queue: [0, 4) the best four, [4, 32) the        */
/* neighbours of the last expanded node.  Warp-wide steps are emulated on     */
/* snapshots so every lane reads the values of before the step.               */
/* ------------------------------------------------------------------------ */
int64_t qvo_nav_entry(const qvo_nav* nav, const float* q, int64_t fallback) {
  enum { L = 4, R = 28, S = 32, WARPS = 4, CHUNK = (R + WARPS - 1) / WARPS };
  const size_t esz = nav->dtype == QVO_FLOAT ? 4 : 1;
  const size_t row = (size_t)nav->dim * esz;
  const uint8_t* data = (const uint8_t*)nav->data;
  const int64_t glen = nav->num_node * (int64_t)nav->max_m;
  uint32_t id[S];
  float dist[S];
  /* init (:82-93): slot 0 = root, the rest empty (id with the visited bit) */
  id[0] = (uint32_t)nav->start;
  dist[0] = qvo_exact_l2(q, data + (size_t)nav->start * row, nav->dtype, nav->dim);
  for (int s = 1; s < S; s++) {
    id[s] = 0xffffffffu;
    dist[s] = INFINITY;
  }
  int idx = 0;
  while (idx != -1) {
    /* expand (:101-104) */
    const uint32_t u = id[idx] & ID_MASK;
    id[idx] |= VISITED;
    /* distance phase (:113-135): warp w takes neighbours [7w, 7w+7) and stops
     * at its first -1; slots past the break keep their values.  The row is
     * read with stride max_m but always 28 wide; past the table's end (where
     * the reference reads outside its array) the slot reads as -1. */
    const int64_t e0 = (int64_t)nav->max_m * (int64_t)u;
    for (int w = 0; w < WARPS; w++) {
      for (int i = w * CHUNK; i < (w + 1) * CHUNK && i < R; i++) {
        const int32_t v = e0 + i < glen ? nav->graph[e0 + i] : -1;
        if (v == -1) break;
        id[i + L] = (uint32_t)v;
        dist[i + L] = qvo_exact_l2(q, data + (size_t)v * row, nav->dtype, nav->dim);
      }
    }
    /* selection phase (:142-182): promote four minima into [0, 4) */
    for (int i = 0; i < L; i++) {
      float cd[S];
      int pos[S];
      const uint32_t prev = i != 0 ? id[i - 1] : 0;
      uint32_t dup_or = 0;
      for (int lane = 0; lane < S; lane++) {
        cd[lane] = dist[lane];
        pos[lane] = lane;
        if (lane < i) {
          cd[lane] = INFINITY;
        } else if (i != 0 && ((id[lane] ^ prev) & ID_MASK) == 0) {
          /* duplicate of the last promoted id: its visited bit joins slot i-1 */
          dup_or |= id[lane];
          dist[lane] = INFINITY;
          cd[lane] = INFINITY;
        }
      }
      if (i != 0) id[i - 1] |= dup_or;
      /* shuffle-down argmin with strict <, offsets 16..1 (:159-167); a lane
       * whose source is past lane 31 reads its own value */
      for (int off = S / 2; off > 0; off /= 2) {
        float od[S];
        int op[S];
        for (int lane = 0; lane < S; lane++) {
          const int src = lane + off < S ? lane + off : lane;
          od[lane] = cd[src];
          op[lane] = pos[src];
        }
        for (int lane = 0; lane < S; lane++) {
          if (od[lane] < cd[lane]) {
            cd[lane] = od[lane];
            pos[lane] = op[lane];
          }
        }
      }
      /* lane 0 swaps slot i with the winner unless their distances are equal
       * (:170-180) */
      const int p = pos[0];
      if (i != p) {
        const float t = dist[i], y = dist[p];
        if (t != y) {
          dist[i] = y;
          dist[p] = t;
          const uint32_t m = id[i];
          id[i] = id[p];
          id[p] = m;
        }
      }
    }
    /* next: first unvisited slot among all 32, kept only below L (:186-191) */
    int x = S;
    for (int s = 0; s < S; s++) {
      if (!(id[s] & VISITED)) {
        x = s;
        break;
      }
    }
    idx = x < L ? x : -1;
  }
  const uint32_t best = id[0] & ID_MASK;
  return best < (uint64_t)nav->num_node ? nav->mapping[best] : fallback;
}

/* ------------------------------------------------------------------------ */
/* One query: persistent_search_kernel body, kernel_q1.cuh:126-704, with the */
/* node fetch served instantly (graph resident in memory), so every issued   */
/* lane is ready on the next pipe iteration.                                  */
/* ------------------------------------------------------------------------ */
static int search_one_impl(const qvo_index* ix, const float* q, const qvo_search_params* p,
                           int32_t* out_ids, float* out_dists, int32_t* out_found,
                           int32_t* out_hops, int32_t* trace, int trace_cap,
                           const int32_t* sr_row, int32_t* sr_step, int32_t* sr_hits);

int qvo_search_one(const qvo_index* ix, const float* q, const qvo_search_params* p,
                   int32_t* out_ids, float* out_dists, int32_t* out_found,
                   int32_t* out_hops) {
  return search_one_impl(ix, q, p, out_ids, out_dists, out_found, out_hops, NULL, 0, NULL, NULL, NULL);
}

int qvo_search_trace(const qvo_index* ix, const float* q, const qvo_search_params* p,
                     int32_t* out_ids, float* out_dists, int32_t* out_found,
                     int32_t* out_hops, int32_t* trace, int trace_cap) {
  const int32_t* row = p->sr_gt ? p->sr_gt : NULL;  /* one query: ground-truth row 0 */
  return search_one_impl(ix, q, p, out_ids, out_dists, out_found, out_hops, trace, trace_cap, row,
                         row ? p->sr_step : NULL, row ? p->sr_hits : NULL);
}

/* count_topk_gt_hits: kernel_helpers.cuh:520-535 -- top-k entries (padding
 * -1 skipped, a repeated id counted each time) found in the ground-truth row. */
static int topk_gt_hits(const int32_t* nns, int topk, const int32_t* gt, int width) {
  int hits = 0;
  for (int i = 0; i < topk; i++) {
    if (nns[i] < 0) continue;
    for (int j = 0; j < width; j++) {
      if (nns[i] == gt[j]) {
        hits++;
        break;
      }
    }
  }
  return hits;
}

static int search_one_impl(const qvo_index* ix, const float* q, const qvo_search_params* p,
                           int32_t* out_ids, float* out_dists, int32_t* out_found,
                           int32_t* out_hops, int32_t* trace, int trace_cap,
                           const int32_t* sr_row, int32_t* sr_step, int32_t* sr_hits) {
  if (sr_row && p->pipe_width != 1) return QVO_EINVAL;
  if (p->topk <= 0 || p->ef_search <= 0 || p->pipe_width < 1 || p->pipe_width > 16)
    return QVO_EINVAL;
  const int W = p->pipe_width;
  const int ef = p->ef_search;
  const int R = ix->max_m;
  const int cap = ef + R + 1;
  qstate s;
  memset(&s, 0, sizeof(s));
  s.ef = ef;
  s.max_m = R;
  s.topk = p->topk;
  s.nid = (uint32_t*)calloc((size_t)cap, sizeof(uint32_t));
  s.ndist = (float*)calloc((size_t)cap, sizeof(float));
  s.tmp_id = (uint32_t*)calloc((size_t)cap, sizeof(uint32_t));
  s.tmp_dist = (float*)calloc((size_t)cap, sizeof(float));
  s.mv_id = (uint32_t*)calloc((size_t)cap, sizeof(uint32_t));
  s.mv_dist = (float*)calloc((size_t)cap, sizeof(float));
  s.mv_pos = (int*)calloc((size_t)cap, sizeof(int));
  s.written = (unsigned char*)calloc((size_t)cap, 1);
  s.nns = (int32_t*)malloc(sizeof(int32_t) * (size_t)p->topk);
  s.tdist = (float*)malloc(sizeof(float) * (size_t)p->topk);
  float* lut = (float*)malloc(sizeof(float) * (size_t)ix->num_chunks * QVO_NUM_PIVOTS);
  float* q_used = (float*)malloc(sizeof(float) * (size_t)ix->dim);
  int rc = QVO_OK;

  qvo_lut_build(ix, q, lut, q_used);
  s.fc = 0;
  s.ctx_size = 0;
  for (int i = 0; i < p->topk; i++) {
    s.tdist[i] = INFINITY;
    s.nns[i] = -1;
  }
  gprune g = {0, 0, INFINITY, INFINITY};
  int step = 0;
  int stop = 0;
  int sr_reached = 0, sr_at = -1, sr_h = 0;
  int32_t lane_req[16];
  int32_t lane_node[16];
  int lane_ready[16];
  /* entry: the nav search on the raw query, else the medoid
   * (kernel_q1.cuh:152-174, 198-205) */
  int64_t entry = p->nav ? qvo_nav_entry(p->nav, q, ix->medoid) : ix->medoid;

  /* boot: kernel_q1.cuh:199-397 */
  rc = merge_data(ix, &s, lut, entry);
  if (rc != QVO_OK) goto done;
  lane_req[0] = visit_select(ix, &s, q_used, entry);
  if (trace && trace_cap > 0) trace[0] = (int32_t)entry;
  step = 1;
  if (gpruning_step(p, &s, &g, step)) {
    stop = 1;
    lane_req[0] = -1;
  }
  if (sr_row && !stop) {
    const int h = topk_gt_hits(s.nns, p->topk, sr_row, p->sr_width);
    if (h >= p->sr_required) {
      sr_reached = 1;
      sr_at = step;
      sr_h = h;
      stop = 1;
      lane_req[0] = -1;
    }
  }
  for (int w = 1; w < W; w++) lane_req[w] = select_next_no_compact(&s);
  for (int w = 0; w < W; w++) {
    lane_ready[w] = (!stop && lane_req[w] != -1);
    lane_node[w] = lane_req[w];
  }

  /* pipe loop: kernel_q1.cuh:407-670 */
  while (!stop) {
    int any = 0;
    for (int w = 0; w < W; w++) any |= lane_ready[w];
    if (!any) break; /* converged: no lane active */
    int ready_now[16];
    for (int w = 0; w < W; w++) ready_now[w] = lane_ready[w];
    for (int w = 0; w < W; w++) {
      if (!ready_now[w]) continue;
      lane_ready[w] = 0; /* status = IDLE (:496) */
      rc = merge_data(ix, &s, lut, lane_node[w]);
      if (rc != QVO_OK) goto done;
      lane_req[w] = visit_select(ix, &s, q_used, lane_node[w]);
      if (trace && step < trace_cap) trace[step] = lane_node[w];
      ++step;
      if (gpruning_step(p, &s, &g, step)) {
        stop = 1;
        lane_req[w] = -1;
      }
      if (sr_row && !stop) {
        const int h = topk_gt_hits(s.nns, p->topk, sr_row, p->sr_width);
        if (h >= p->sr_required) {
          sr_reached = 1;
          sr_at = step;
          sr_h = h;
          stop = 1;
          lane_req[w] = -1;
        }
      }
    }
    if (stop) break;
    /* phase 1: idle lanes that were not served this iteration (:622-630) */
    for (int w = 0; w < W; w++) {
      if (!ready_now[w] && !lane_ready[w]) lane_req[w] = select_next_no_compact(&s);
    }
    /* phase 2: issue (:635-653) */
    for (int w = 0; w < W; w++) {
      if (lane_req[w] != -1) {
        lane_ready[w] = 1;
        lane_node[w] = lane_req[w];
      }
    }
  }

done:
  if (rc == QVO_OK) {
    for (int i = 0; i < p->topk; i++) {
      out_ids[i] = s.nns[i];
      out_dists[i] = s.tdist[i];
    }
    if (out_found) *out_found = s.fc;
    if (out_hops) *out_hops = step;
    if (sr_row) {
      if (sr_step) *sr_step = sr_reached ? sr_at : -1;
      if (sr_hits) *sr_hits = sr_reached ? sr_h : topk_gt_hits(s.nns, p->topk, sr_row, p->sr_width);
    }
  }
  free(s.nid); free(s.ndist); free(s.tmp_id); free(s.tmp_dist);
  free(s.mv_id); free(s.mv_dist); free(s.mv_pos); free(s.written);
  free(s.nns); free(s.tdist); free(lut); free(q_used);
  return rc;
}

static double wall_seconds(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int qvo_search(const qvo_index* ix, const float* queries, int64_t nq,
               const qvo_search_params* p, int threads, int32_t* ids,
               float* dists, int32_t* found, int32_t* hops) {
  return qvo_search_timed(ix, queries, nq, p, threads, ids, dists, found, hops, NULL);
}

int qvo_search_timed(const qvo_index* ix, const float* queries, int64_t nq,
                     const qvo_search_params* p, int threads, int32_t* ids,
                     float* dists, int32_t* found, int32_t* hops, double* seconds) {
  int status = QVO_OK;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_num_procs();
#pragma omp parallel for schedule(dynamic, 4) num_threads(threads)
#endif
  for (int64_t i = 0; i < nq; i++) {
    const double t0 = seconds ? wall_seconds() : 0.0;
    const int32_t* sr_row = p->sr_gt ? p->sr_gt + (i % p->sr_count) * (int64_t)p->sr_width : NULL;
    int rc = search_one_impl(ix, queries + i * (int64_t)ix->dim, p,
                             ids + i * p->topk, dists + i * p->topk,
                             found ? found + i : NULL, hops ? hops + i : NULL, NULL, 0, sr_row,
                             sr_row && p->sr_step ? p->sr_step + i : NULL,
                             sr_row && p->sr_hits ? p->sr_hits + i : NULL);
    if (seconds) seconds[i] = wall_seconds() - t0;
    if (rc != QVO_OK) {
#ifdef _OPENMP
#pragma omp critical
#endif
      { if (status == QVO_OK) status = rc; }
    }
  }
  (void)threads;
  return status;
}

/* ------------------------------------------------------------------------ */
/* calc_recall: bin/common/recall.hpp:44-62.                                  */
/* ------------------------------------------------------------------------ */
double qvo_recall(const int32_t* results, const int32_t* gt, int64_t nq,
                  int gt_width, int k) {
  int64_t hits = 0;
  for (int64_t i = 0; i < nq; i++) {
    const int32_t* g = gt + i * gt_width;
    for (int j = 0; j < k; j++) {
      int32_t r = results[i * k + j];
      for (int t = 0; t < k; t++) {
        if (g[t] == r) { hits++; break; }
      }
    }
  }
  return (double)hits / (double)(nq * (int64_t)k);
}

/* ------------------------------------------------------------------------ */
/* ADC + top-k microbenchmark: for each s the ADC above, top-k under          */
/* (dist, s) -- identical to the reference's stable first-found-wins insert  */
/* (kernel_helpers.cuh:65-104) applied in order s = 0, 1, ...                */
/* ------------------------------------------------------------------------ */
void qvo_adc_topk(const float* lut, int num_chunks, const uint8_t* codes,
                  const int32_t* ids, int64_t nids, int k, int32_t* out_ids,
                  float* out_dists, double* dist_sum) {
  int fc = 0;
  double sum = 0.0;
  for (int i = 0; i < k; i++) {
    out_ids[i] = -1;
    out_dists[i] = INFINITY;
  }
  for (int64_t s = 0; s < nids; s++) {
    float d = qvo_adc(lut, num_chunks, codes + (int64_t)ids[s] * num_chunks);
    sum += (double)d;
    if (fc < k || d < out_dists[k - 1]) {
      int pos = 0;
      while (pos < fc && out_dists[pos] <= d) pos++;
      int ns = fc < k ? fc + 1 : k;
      for (int i = ns - 1; i > pos; i--) {
        out_dists[i] = out_dists[i - 1];
        out_ids[i] = out_ids[i - 1];
      }
      out_dists[pos] = d;
      out_ids[pos] = ids[s];
      fc = ns;
    }
  }
  if (dist_sum) *dist_sum = sum;
}

/* ------------------------------------------------------------------------ */
/* Brute-force ground truth in float64 (ties broken by smaller id).          */
/* ------------------------------------------------------------------------ */
void qvo_ground_truth(const void* base, int dtype, int64_t n, int dim,
                      const float* queries, int64_t nq, int k, int threads,
                      int32_t* gt_ids, float* gt_dists) {
  size_t esz = dtype == QVO_FLOAT ? 4 : 1;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_num_procs();
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
  for (int64_t qi = 0; qi < nq; qi++) {
    const float* q = queries + qi * dim;
    double* bd = (double*)malloc(sizeof(double) * (size_t)k);
    int64_t* bi = (int64_t*)malloc(sizeof(int64_t) * (size_t)k);
    int cnt = 0;
    for (int64_t x = 0; x < n; x++) {
      const void* row = (const uint8_t*)base + (size_t)x * dim * esz;
      double acc = 0.0;
      for (int i = 0; i < dim; i++) {
        double diff = (double)q[i] - (double)elem_as_float(row, dtype, i);
        acc += diff * diff;
      }
      if (cnt < k || acc < bd[cnt - 1] || (acc == bd[cnt - 1] && x < bi[cnt - 1])) {
        int pos = cnt < k ? cnt : k - 1; /* slot freed for the new entry */
        while (pos > 0 && (bd[pos - 1] > acc || (bd[pos - 1] == acc && bi[pos - 1] > x))) {
          bd[pos] = bd[pos - 1];
          bi[pos] = bi[pos - 1];
          pos--;
        }
        bd[pos] = acc;
        bi[pos] = x;
        if (cnt < k) cnt++;
      }
    }
    for (int j = 0; j < k; j++) {
      gt_ids[qi * k + j] = j < cnt ? (int32_t)bi[j] : -1;
      if (gt_dists) gt_dists[qi * k + j] = j < cnt ? (float)bd[j] : INFINITY;
    }
    free(bd);
    free(bi);
  }
  (void)threads;
}
