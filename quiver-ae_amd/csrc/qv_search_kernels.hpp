// qv_search_kernels.hpp -- the persistent beam-search kernels (device code),
// shared by the translation units that instantiate them: qv_search.hip (one
// neighbour per lane, beams up to 448 entries), qv_search_deep.hip (beams up
// to 1024 entries) and qv_search_r128.hip (two neighbours per lane, R <= 128).
// The reference path each part follows is cited where it is defined.
#pragma once

#include <cstdint>

#include "qv_common.hpp"
#include "qv_device.hpp"

#include <type_traits>

namespace qv {
namespace sk {

using namespace qv::dev;

struct SearchArgs {
  // index (HBM)
  const uint8_t* pages;
  const uint8_t* codes;
  const float* centroid;
  const float* pivots_t;
  const int32_t* chunk_off;
  int64_t num_points;
  int64_t nodes_per_page;
  uint64_t npp_magic;              // page = (v * npp_magic) >> npp_shift, exact for 0 <= v < 2^31
  int32_t npp_shift;
  int64_t node_size;
  int64_t data_size;
  int32_t dim;
  int32_t num_chunks;
  int32_t max_m;
  int32_t medoid;
  // queries / params
  const float* queries;
  int32_t nq;
  int32_t topk;
  int32_t ef;
  int32_t pipe_w;
  int32_t early_exit;
  int32_t warmup;
  int32_t patience;
  // outputs (device)
  int32_t* out_ids;
  float* out_dists;
  int32_t* out_found;
  int32_t* out_hops;
  int32_t* out_stopped;
  int32_t* out_evals;              // neighbour distance evaluations per query
  uint64_t* t_start;
  uint64_t* t_end;
  // dispatch
  int32_t* counters;               // [0] next ticket, [1] done count, [2] error bits, [3] ring
                                   // position, [4] queries that entered tail mode
  const int32_t* feed_count;       // host-coherent, may be null (then nq)
  const int32_t* terminate;        // host-coherent, may be null
  int32_t* ring;                   // host-coherent completion ring, may be null
  uint64_t spin_limit_ticks;       // watchdog on feed waits (100 MHz ticks)
  uint64_t* feed_mirror;           // kFeedLines words, kFeedStride apart: (epoch << 32) | feed
  uint32_t feed_epoch;             // this search's epoch (a word of another epoch reads as 0)
  // navigation graph for the per-query entry node (nav_data null: the medoid)
  const uint8_t* nav_data;
  const int32_t* nav_graph;
  const int32_t* nav_map;
  int64_t nav_nodes;
  int32_t nav_max_m;
  int32_t nav_start;
  // optional record of expanded nodes (graph construction)
  int32_t* rec_ids;
  float* rec_dists;
  int32_t rec_cap;
  // per-step recall (pipe width 1): query q stops once sr_required of its
  // top-k ids appear in ground-truth row q % sr_count (sr_width <= 256 ids);
  // sr_gt null: off
  const int32_t* sr_gt;
  int32_t sr_width;
  int32_t sr_count;
  int32_t sr_required;
  int32_t* sr_step;                // [nq] step at which it was reached, -1 if never
  int32_t* sr_hits;                // [nq] hits then (else at the end)
  // neighbour code table (optional, null: off): node v's neighbours' code
  // rows, slot order, at nbr_codes + v * max_m * num_chunks (zero past its degree)
  const uint8_t* nbr_codes;
  // shared pivots: [gridDim.x] waves of each workgroup that have ended, zero
  // at launch (null: no tail mode; never set for one-wave workgroups)
  int32_t* wg_done;
};

enum : int32_t { kErrSpinTimeout = 1 };

// Device copies of the host's feed word: one 8-byte word per line, the lines
// 4352 bytes apart so that the waiting waves' reads spread over many memory
// channels instead of queueing at one.
constexpr int kFeedLines = 64;  // one per lane of the publishing wave
constexpr int64_t kFeedStride = 4352 / 8;  // in 8-byte words
constexpr int64_t kFeedMirrorBytes = kFeedLines * kFeedStride * 8;

// Workgroups of a shared-pivot launch whose ended waves are counted for
// tail mode (one 32-bit count each, after the 64 bytes of launch counters).
constexpr int kMaxTailWorkgroups = 4096;

// 32-bit words ahead of the per-query counts in the host's pinned staging
// buffer: the launch counters copied back after a search.
constexpr int kStageHead = 8;

// Dynamic LDS carve-up of one query (one wave), shared by the kernel and its
// launcher.  Q = beam positions per lane: the register beam holds Q * 64 >= ef
// entries, the LDS beam cap of them (beam_cap).  With a per-query LUT (lut) the
// table comes first; the shared-pivot kernel has none, and when every query
// element the exact distance needs fits the lanes' registers
// (dim <= 32 kVecPre) its beam overlays both query copies, qc and qu, which
// are only read once, into registers (load_query_dpp, load_query_pre),
// before the first hop.
struct LdsPlan {
  int lut_off, qc_off, qu_off, beam_off, count_off, wide_off, total;
};

// Top-k entries a wave holds in its registers: entry i in lane i.  The
// per-query-LUT kernel keeps entries 64 .. k - 1 of a larger k in LDS after
// the rest of the query's area (wide_topk entries of 8 bytes: the distances,
// then the ids); the shared-pivot kernel takes k <= 64 only.
constexpr int kRegTopk = 64;
__host__ __device__ inline int wide_topk(int topk) { return topk > kRegTopk ? (topk - kRegTopk + 7) & ~7 : 0; }

// LDS beam entries: Q * 64 with the per-query LUT (its table, not the beam,
// limits the queries per CU); ef rounded up to 8 with shared pivots, where the
// beam's LDS decides how many queries a CU holds.
__host__ __device__ inline int beam_cap(int ef, int Q, bool lut) { return lut ? Q * kWave : (ef + 7) & ~7; }

// Whether a merge counts its surviving candidates per beam rank in LDS (one
// word per beam position, after the beam): the per-query-LUT kernel up to
// Q = 7, where the counts still leave room for 4 queries of 32-chunk LUTs per
// CU.  The other kernels add the candidates one at a time.
__host__ __device__ constexpr bool rank_counts(bool lut, int Q) { return lut && Q <= 7; }

__host__ __device__ inline LdsPlan lds_plan(int num_chunks, int dim, int Q, bool lut, int ef, int topk) {
  LdsPlan p;
  p.lut_off = 0;
  p.qc_off = p.lut_off + (lut ? num_chunks * kPivots * 4 : 0);
  const int dpad = (dim + 3) & ~3;
  p.qu_off = p.qc_off + dpad * 4;
  const bool overlay = !lut && dim <= 32 * kVecPre;
  p.beam_off = overlay ? p.qc_off : (p.qu_off + dpad * 4 + 15) & ~15;
  const int beam_bytes = beam_cap(ef, Q, lut) * 8;
  p.count_off = p.beam_off + beam_bytes;  // (rank_counts: no overlay)
  p.total = p.beam_off + (overlay && 2 * dpad * 4 > beam_bytes ? 2 * dpad * 4 : beam_bytes) +
            (rank_counts(lut, Q) ? beam_cap(ef, Q, lut) * 4 : 0);
  p.wide_off = p.total;
  if (lut) p.total += wide_topk(topk) * 8;
  return p;
}

// Shared-pivot kernel: the PQ pivots chunk-major, [chunk m][code c][SC dims]
// (entry (m, c) at float (m * 256 + c) * SC), ahead of the per-wave query
// areas.  The SC floats one LUT entry needs are one aligned vector read, and
// lanes reading different codes of one chunk hit consecutive 4 SC-byte slots,
// so rows need no padding against bank conflicts.
__host__ __device__ inline int piv_bytes(int dim) { return kPivots * dim * 4; }

using KernelFn = void (*)(SearchArgs);

// Beam positions per lane of the kernels for ef above 1024.
constexpr int kXlQ = 32;

// Waves (queries) one shared-pivot workgroup holds at most, by beam positions
// per lane and neighbour slots per lane: 16 (128 registers per wave), or 8
// (256) for beams of more than 7 positions per lane and for two slots.
__host__ __device__ constexpr int sp_max_waves(int Q, int NPL) { return Q <= 7 && NPL == 1 ? 16 : 8; }

// Kernels instantiated in qv_search_r128.hip (two neighbour slots per lane,
// Q rounded up to 1, 2, 4, 7, 10 or 16) and qv_search_deep.hip (one slot per
// lane, Q = 10 or 16); null for a combination they do not hold.
KernelFn pick_kernel_r128(int dtype, int Q, int M);
KernelFn pick_kernel_sp_r128(int dtype, int Q, int M);
KernelFn pick_kernel_deep(int dtype, int Q, int M);
KernelFn pick_kernel_sp_deep(int dtype, int Q, int M);
// Per-query-LUT kernels for a top-k above 64 (qv_search_wide.hip): Q = 2, 4,
// 7, 10 or 16 (from wide_beam_chunks), one or two neighbour slots per lane.
KernelFn pick_kernel_wide(int dtype, int Q, int M, int npl);
__host__ __device__ inline int wide_beam_chunks(int ef) {
  return ef <= 128 ? 2 : (ef <= 256 ? 4 : (ef <= 448 ? 7 : (ef <= 640 ? 10 : (ef <= 1024 ? 16 : kXlQ))));
}
// Per-query-LUT kernels for ef in (1024, 2048] (qv_search_xl.hip): Q = 32,
// any top-k.
KernelFn pick_kernel_xl(int dtype, int M, int npl, bool wide);

}  // namespace sk
}  // namespace qv

namespace {

using namespace qv::sk;

// Registers holding the start of a node record (see Query::fetch): NPL
// neighbour slots per lane (lane l holds neighbours l and l + 64).
template <class T, int NPL>
struct NodeRec {
  // raw vector elements (load_vec_pre); bytes stay 8-bit values, so where two
  // loads of them meet, the registers join without a zero-extension
  using Raw = std::conditional_t<sizeof(T) == 1, uint8_t, uint32_t>;
  int deg;
  uint32_t nbr[NPL];
  Raw xv[kVecPre];
};

// What a hop reads of its node's record, taken out of the registers the
// record's loads wrote (Query::take) once they have arrived: the degree, this
// lane's neighbour ids (0 past the degree) and this lane's sum over its
// first vector elements for the exact distance.
template <int NPL>
struct Taken {
  int deg;
  uint32_t nbr[NPL];
  float part;
};

// SC = 0: per-query LUT in LDS; SC > 0: LUT entries recomputed from the
// shared pivots (chunks of SC dimensions).  NPL = 1: R <= 64, lane l owns
// neighbour l; NPL = 2: R <= 128, lane l also owns neighbour l + 64.  WK: a
// top-k above 64 (per-query LUT only), entries past the 64th in LDS.
template <class T, int Q, int MC, int SC, int NPL, bool WK = false>
struct Query {
  static_assert(NPL == 1 || NPL == 2, "one or two neighbours per lane");
  static_assert(!WK || SC == 0, "a top-k above 64 runs on the per-query-LUT kernel");
  using Rec = NodeRec<T, NPL>;
  using Tk = Taken<NPL>;
  const SearchArgs& a;
  float* lut;
  const float* piv;  // shared pivots (SC > 0)
  float* qc;
  float* qu;
  float quv[kVecPre];  // qu elements of this lane for the exact distance
  // q' for the shared-pivot ADC, 16 elements per register (load_query_dpp)
  static constexpr int kQd = SC > 0 ? (MC * SC + 15) / 16 : 1;
  float qd[kQd];
  uint64_t* beam;
  // surviving candidates per beam rank (kCounts), zero between merges
  uint32_t* rcount;
  static constexpr bool kCounts = rank_counts(SC == 0, Q);
  // 8-ary rank search (needs cap = 64 Q); at Q = 1 the 4-ary one also takes
  // two LDS round trips, with fewer reads.
  static constexpr bool kRank8 = kCounts && Q >= 2;
  int sz;        // beam size (ctx.size)
  int cap;       // LDS beam entries (beam_cap >= ef)
  // The beam in registers, chunk-major (lane l holds positions [l Q, l Q + Q),
  // kPadKey at and beyond sz), and its first unvisited entry u with key bu
  // (INT32_MAX and ~0 when every entry is visited).  LDS holds the same beam
  // for the scatter of each merge.  Which entries are unvisited is um's to
  // say (bit k: slot k of this lane, below sz): marking an entry visited
  // clears its bit only, and the visited bits of ck are brought up to date
  // from um when a merge writes the beam back.  At Q = 1 marking clears the
  // visited bit of ck itself and um is derived from it when needed (one slot
  // per lane: that is as cheap, and the scatter needs no restoring).
  uint64_t ck[Q];
  uint32_t um;
  int u;
  uint64_t bu;
  float td;      // top-k entry of this lane
  int32_t ti;
  // (WK) top-k entries 64 .. topk - 1 in LDS
  float* wd;
  int32_t* wi;
  int fc;        // found count
  int evals;     // ADC evaluations so far
  float last_e;  // exact distance of the node expanded by the last hop
  // The beam's entry at ef - 1 when the beam is full (~0 before): candidates
  // at or above it cannot enter.  Only merges change it; marking an entry
  // visited does not matter here (a candidate's key equals an entry's only
  // with the same id, which is not below it either way).
  uint64_t lastk;
  // (kRank8) the beam's entries at 64 j - 1, j = 1 .. Q - 1, from the
  // register copy (kPadKey past sz), wave-uniform: the first level of the
  // rank search, renewed whenever the beam changes.
  uint64_t pk[Q > 1 ? Q - 1 : 1];

  // Tail mode (shared pivots, 32 chunks of 4 dims): once this wave is the
  // last of its workgroup with a query -- the ticket queue is empty and its
  // workgroup mates have ended -- nothing else reads the pivot table, so the
  // wave builds its own LUT over it (enter_tail) and finishes the query with
  // table lookups instead of recomputing every entry: a lone wave's hop then
  // costs what it costs in the per-query-LUT kernel.  The search loop has a
  // copy for tail mode (hop<PF, true>), so the other copy keeps its hop.
  // (Not at Q = 1: a beam of at most 64 ends its queries soon, and the
  // probe's registers cost more there than the tail saves.)
  static constexpr bool kTail = SC == 4 && MC == 32 && NPL == 1 && Q > 1;

  // The shared-pivot kernels serve dim = MC SC only (uniform chunks).
  static constexpr int kD = SC > 0 ? MC * SC : 0;
  // Loop-invariant byte offsets of this lane's loads inside a record: its
  // neighbour slot (past the degree word) and its first vector element.
  uint32_t off_nbr[NPL], off_x;
  // (kD == 0) byte offsets of this lane's first vector elements,
  // min((lane & 31) + 32 k, dim - 1)
  uint32_t off_xk[kD > 0 ? 1 : kVecPre];
  uint32_t off_blk;  // this lane's row in a node's neighbour-code block

  // smem: this query's LDS area.
  __device__ Query(const SearchArgs& args, char* smem, const float* pivots_lds)
      : a(args), piv(pivots_lds), sz(0), um(0), u(INT32_MAX), bu(~0ull), td(__int_as_float(0x7f800000)), ti(-1), fc(0),
        evals(0), lastk(~0ull) {
#pragma unroll
    for (int k = 0; k < Q; k++) ck[k] = kPadKey;
#pragma unroll
    for (int j = 0; j < Q - 1; j++) pk[j] = kPadKey;
    LdsPlan pl = lds_plan(a.num_chunks, a.dim, Q, SC == 0, a.ef, a.topk);
    cap = beam_cap(a.ef, Q, SC == 0);
    wd = reinterpret_cast<float*>(smem + pl.wide_off);
    wi = reinterpret_cast<int32_t*>(wd + wide_topk(a.topk));
    lut = reinterpret_cast<float*>(smem + pl.lut_off);
    qc = reinterpret_cast<float*>(smem + pl.qc_off);
    qu = reinterpret_cast<float*>(smem + pl.qu_off);
    beam = reinterpret_cast<uint64_t*>(smem + pl.beam_off);
    rcount = reinterpret_cast<uint32_t*>(smem + pl.count_off);
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < NPL; j++)  // slots >= max_m are masked by the degree
      off_nbr[j] = 4u * (uint32_t)(1 + min(lane + kWave * j, a.max_m - 1));
    off_x = (uint32_t)(lane & 31) * (uint32_t)sizeof(T);
    if constexpr (kD == 0) {
#pragma unroll
      for (int k = 0; k < kVecPre; k++)
        off_xk[k] = (uint32_t)min((lane & 31) + 32 * k, a.dim - 1) * (uint32_t)sizeof(T);
    }
    off_blk = (uint32_t)(min(lane, a.max_m - 1) * a.num_chunks);
  }

  // Node v's neighbour-code block (this lane's row at off_blk).
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t block(int32_t v) const {
    return buf_at(a.nbr_codes + (int64_t)v * (a.max_m * a.num_chunks));
  }

  __device__ __forceinline__ const uint8_t* record(int32_t v) const {
    const int64_t page = (int64_t)(((uint64_t)(uint32_t)v * a.npp_magic) >> a.npp_shift);
    const int64_t slot = (int64_t)v - page * a.nodes_per_page;
    return a.pages + page * 4096 + slot * a.node_size;
  }

  // Requests the parts of v's record a hop reads: degree, the max_m neighbour
  // slots (inside the record) and the first vector elements.  Only vector
  // loads are used, so waits on LDS traffic never wait for these.
  __device__ __forceinline__ void fetch(int32_t v, int lane, Rec& nr) const {
    const uint8_t* rec = record(v);
    const __amdgpu_buffer_rsrc_t r = buf_at(rec);
    const int ds = (int)a.data_size;  // a record is under 4 KB
    nr.deg = (int)__builtin_amdgcn_raw_buffer_load_b32(r, 0, ds, 0);
#pragma unroll
    for (int j = 0; j < NPL; j++) nr.nbr[j] = __builtin_amdgcn_raw_buffer_load_b32(r, (int)off_nbr[j], ds, 0);
    if constexpr (kD > 0)
      load_vec_pre_buf<T, kD>(r, off_x, nr.xv);
    else
      load_vec_pre_offs<T>(r, off_xk, nr.xv);
  }

  // The values a hop reads first from the record in nr.  Taken at the end
  // of the hop that requested the record, they leave nr free for the next
  // request: a record still in nr when the next one is requested into other
  // registers has to be copied over at the end of the loop, and the copy
  // waits for every load requested before it, the next code rows included.
  __device__ __forceinline__ void take(const Rec& nr, Tk& tk, int lane) const {
    // every load of the record is issued before the first wait for one
    __builtin_amdgcn_sched_barrier(0);
    tk.deg = read_lane_i32(nr.deg, 0);
#pragma unroll
    for (int j = 0; j < NPL; j++) tk.nbr[j] = lane + kWave * j < tk.deg ? nr.nbr[j] : 0u;
    if constexpr (kD > 0)
      tk.part = exact_lane_fixed<T, kD>(nr.xv, quv);
    else
      tk.part = exact_lane_pre<T>(nr.xv, quv, a.dim, lane);
  }

  // Exact distance of v from its lanes' sums (part) and the top-k insert
  // (the reference's second warp).
  __device__ __forceinline__ void exact_and_topk(int32_t v, float part, const uint8_t* rec, int lane) {
    float e;
    if constexpr (kD > 0)
      e = exact_reduce(part, lane);
    else
      e = exact_l2_rest<T>(part, rec, qu, a.dim, lane);
    last_e = e;
    if constexpr (WK) {
      wide_insert(e, v, lane);
      return;
    }
    const float dlast = read_lane_f32(td, a.topk - 1);
    if (fc < a.topk || e < dlast) topk_insert(td, ti, fc, a.topk, e, v);
  }

  // Top-k insert for k > 64 (retset_push_32, gpu_primitives.cuh:99-138; the
  // same order as topk_insert: after every entry <= e, the entry at k - 1
  // dropping out of a full list), called for every expansion; it applies the
  // fc < k || e < D[k - 1] guard itself.  Entries 0 .. 63 are the lanes'
  // registers, entries 64 .. k - 1 the LDS list wd / wi.  The LDS part moves
  // up one place from the insert position in chunks of 64, the highest chunk
  // first, so that every entry is read before the write that replaces it;
  // lane 63's register entry moves to LDS entry 0 when the insert lands in
  // the registers.
  __device__ __forceinline__ void wide_insert(float e, int32_t v, int lane) {
    const int k = a.topk;
    const int f = read_lane_i32(fc, 0);  // equal in every lane
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (f >= k && !(e < wd[k - kRegTopk - 1])) return;
    int pos = __popcll(__ballot(lane < min(f, kRegTopk) && td <= e));
    const int fx = f - kRegTopk;  // LDS entries in use
    if (pos == kRegTopk) {
      for (int b = 0; b < fx; b += kWave) {
        const int j = b + lane;
        const int c = __popcll(__ballot(j < fx && wd[j] <= e));
        pos += c;
        if (c < kWave) break;  // sorted: the rest are above e
      }
    }
    const int ns = min(f + 1, k);
    const int nx = ns - kRegTopk;  // LDS entries after the insert
    if (nx > 0) {
      const float r63d = read_lane_f32(td, kRegTopk - 1);
      const int32_t r63i = read_lane_i32(ti, kRegTopk - 1);
      const int lo = max(pos - kRegTopk, 0);  // first LDS entry that changes
      for (int b = (nx - 1) & ~(kWave - 1); b >= 0 && b + kWave > lo; b -= kWave) {
        const int j = b + lane;
        const bool w = j >= lo && j < nx;
        float dv = e;
        int32_t iv = v;
        if (w && kRegTopk + j != pos) {
          if (j == 0) {
            dv = r63d;
            iv = r63i;
          } else {
            dv = wd[j - 1];
            iv = wi[j - 1];
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (w) {
          wd[j] = dv;
          wi[j] = iv;
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      }
    }
    if (pos < kRegTopk) {
      int fr = min(f, kRegTopk);
      topk_insert(td, ti, fr, kRegTopk, e, v);
    }
    fc = ns;
  }

  // Top-k entry k - 1's distance (+inf while fewer than k are found), the
  // same in every lane.
  __device__ __forceinline__ float kth_dist() const {
    if constexpr (WK) {
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      const float d = wd[a.topk - kRegTopk - 1];
      return read_lane_i32(fc, 0) >= a.topk ? d : __int_as_float(0x7f800000);
    }
    return read_lane_f32(td, a.topk - 1);
  }

  // Top-k entry i's id (-1: not found yet), the same in every lane.
  __device__ __forceinline__ int32_t id_at(int i) const {
    if constexpr (WK) {
      if (i >= kRegTopk) {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const int32_t id = wi[i - kRegTopk];
        return i < read_lane_i32(fc, 0) ? id : -1;
      }
    }
    return read_lane_i32(ti, i);
  }

  // Entries 64 .. k - 1 of the query's results (k > 64), -1 / +inf past fc.
  __device__ __forceinline__ void write_wide(int32_t qid, int lane) const {
    if constexpr (WK) {
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      const int f = read_lane_i32(fc, 0);
      int32_t* const oi = a.out_ids + (int64_t)qid * a.topk + kRegTopk;
      float* const od = a.out_dists + (int64_t)qid * a.topk + kRegTopk;
      for (int j = lane; j < a.topk - kRegTopk; j += kWave) {
        const bool ok = kRegTopk + j < f;
        const int32_t id = wi[j];
        const float d = wd[j];
        oi[j] = ok ? id : -1;
        od[j] = ok ? d : __int_as_float(0x7f800000);
      }
    }
  }

  // One expansion of node v: persistent_merge_data (kernel_helpers.cuh:232-357)
  // followed by persistent_visit_select_dualwarp (kernel_helpers.cuh:422-489).
  // tk holds what was taken from v's record (fetch, take).  Returns the
  // selected node or -1.  PF says which node's record the hop requests into
  // nr and takes into tk at its end: 0 none, 1 the speculated successor
  // (below; with PF = 1 the selected node's record is also requested as soon
  // as the merge knows it, when the guess missed), 2 the caller's nxt (the
  // pipe lanes' next expansion; -1: not known, v's record again).
  //
  // With PF, cr carries code rows from one hop to the next: when `have`, cr
  // holds (or is loading) v's neighbours' rows, requested by the previous hop.
  // A hop that guesses its successor (the beam's first unvisited entry, spec)
  // requests that node's record at its start and, once the ADC no longer
  // needs cr, that node's code rows, so the next hop's rows are in flight
  // through this hop's merge; `have` is set when the guess was the node
  // selected.  PF = 2 does the same for nxt, and `have` says nxt's rows are
  // in cr.  Only loads move: every result is the same.
  static constexpr bool kRows = MC > 0 && MC % 16 == 0;  // code rows in registers (adc_load)

  // TL: the wave is in tail mode (kTail): the ADC reads its own LUT.
  template <int PF, bool TL = false>
  __device__ __forceinline__ int32_t hop(int32_t v, Tk& tk, Rec& nr, CodeRow<MC>& cr, bool& have,
                                         int32_t nxt = -1) {
    if constexpr (NPL == 2) return hop2<PF == 1>(v, tk, nr);
    const int lane = opaque_lane();
    const int deg = tk.deg;
    evals += deg;
    const bool has = lane < deg;
    const uint32_t nbr = tk.nbr[0];
    const uint8_t* rec = kD == 0 && a.dim > 32 * kVecPre ? record(v) : nullptr;
    // With PF, the next node is most often the beam's first unvisited entry
    // (whenever no new candidate beats it), so its record is requested right
    // after this hop's code rows, and the merge only requests another record
    // when a candidate wins.
    const bool spec = PF == 1 && u < sz;

    // ADC gather-sum over the neighbour's code row (LUT in LDS); the code rows
    // are in flight while the exact distance of v is computed.  Lanes without
    // a neighbour read code row 0 and discard the sum.
    float d;
    // With the neighbour-code table a node's rows are one contiguous block
    // whose address needs no neighbour ids, so the guessed successor's rows
    // are requested without waiting for its record, and after a wrong guess
    // the chosen node's rows follow its record at once.
    const bool blk = a.nbr_codes != nullptr;
    if constexpr (kRows) {
      if (!(PF != 0 && have)) {
        if (blk)
          adc_load<MC>(cr, block(v), off_blk);
        else
          adc_load<MC>(cr, a.codes, nbr);
      }
      // Issued on every hop (v's own record when there is no node to
      // request), as are the rows below, so every path reaches each wait with
      // the same loads in flight: the compiler's wait for the code rows then
      // leaves the record outstanding, and the take's for the record leaves
      // the next rows.
      if constexpr (PF == 1) fetch(spec ? (int32_t)key_id(bu) : v, lane, nr);
      if constexpr (PF == 2) fetch(nxt >= 0 ? nxt : v, lane, nr);
      exact_and_topk(v, tk.part, rec, lane);
      if constexpr (SC > 0) {
        if constexpr (kTail && TL)
          d = adc_sum_at0<MC, 1024>(cr);  // the tail LUT: chunk m's entries 4 KB apart
        else
          d = adc_recompute<MC, SC, kQd>(cr, qd);
      } else {
        d = adc_sum_at0<MC>(cr);
      }
      // the next node's code rows (lanes past its degree read row 0): the
      // guessed successor's (PF = 1) or nxt's (PF = 2)
      if constexpr (PF != 0) {
        const bool go = PF == 1 ? spec : nxt >= 0;
        if (blk) {
          adc_load<MC>(cr, block(go ? (PF == 1 ? (int32_t)key_id(bu) : nxt) : v), off_blk);
        } else {
          const int ndeg = read_lane_i32(nr.deg, 0);
          adc_load<MC>(cr, a.codes, lane < ndeg ? nr.nbr[0] : 0u);
        }
      }
    } else {
      if (PF == 1 && spec) fetch((int32_t)key_id(bu), lane, nr);
      if (PF == 2 && nxt >= 0) fetch(nxt, lane, nr);
      d = adc_row<MC>(a.codes + (int64_t)nbr * a.num_chunks, lut, a.num_chunks);
      exact_and_topk(v, tk.part, rec, lane);
    }
    const uint64_t nkey = has ? make_key(d, nbr, false) : sentinel_key(lane);
    bool hit = false;
    const int32_t nx = merge_select<true, PF == 1, kRows>(nkey, has, lane, nr, spec, bu, hit, &cr);
    if constexpr (PF == 1 && kRows) have = hit || (blk && nx >= 0);
    if constexpr (PF == 2 && kRows) have = nxt >= 0;
    if constexpr (PF != 0) take(nr, tk, lane);
    return nx;
  }

  // hop with two neighbours per lane (R <= 128): the same expansion with the
  // candidates merged as two batches of 64, neighbours 0-63 first without a
  // selection, then 64-127 with it.  The first ef entries of
  // (first ef of beam U A) U B are the first ef of beam U A U B; a B
  // neighbour whose entry A pushed out of the beam would have landed at or
  // beyond ef anyway, and no id repeats within one adjacency list.  The
  // guessed successor is the first unvisited entry before A (its record is
  // requested at the start), compared by key after B.
  template <bool PF>
  __device__ __forceinline__ int32_t hop2(int32_t v, Tk& tk, Rec& nr) {
    const int lane = opaque_lane();
    const int deg = tk.deg;
    evals += deg;
    const bool has0 = lane < deg, has1 = lane + kWave < deg;
    const uint32_t nbr0 = tk.nbr[0], nbr1 = tk.nbr[1];
    const uint8_t* rec = kD == 0 && a.dim > 32 * kVecPre ? record(v) : nullptr;
    const bool spec = PF && u < sz;
    const uint64_t spec_key = bu;
    float d0, d1;
    if constexpr (MC > 0 && MC % 16 == 0) {
      CodeRow<MC> c0, c1;
      adc_load<MC>(c0, a.codes, nbr0);
      adc_load<MC>(c1, a.codes, nbr1);
      if constexpr (PF) fetch(spec ? (int32_t)key_id(bu) : v, lane, nr);
      exact_and_topk(v, tk.part, rec, lane);
      if constexpr (SC > 0) {
        d0 = adc_recompute<MC, SC, kQd>(c0, qd);
        d1 = adc_recompute<MC, SC, kQd>(c1, qd);
      } else {
        d0 = adc_sum_at0<MC>(c0);
        d1 = adc_sum_at0<MC>(c1);
      }
    } else {
      if (PF && spec) fetch((int32_t)key_id(bu), lane, nr);
      d0 = adc_row<MC>(a.codes + (int64_t)nbr0 * a.num_chunks, lut, a.num_chunks);
      d1 = adc_row<MC>(a.codes + (int64_t)nbr1 * a.num_chunks, lut, a.num_chunks);
      exact_and_topk(v, tk.part, rec, lane);
    }
    const uint64_t k0 = has0 ? make_key(d0, nbr0, false) : sentinel_key(lane);
    const uint64_t k1 = has1 ? make_key(d1, nbr1, false) : sentinel_key(lane + kWave);
    bool hit = false;
    merge_select<false, false>(k0, has0, lane, nr, false, spec_key, hit);
    const int32_t nx = merge_select<true, PF>(k1, has1, lane, nr, spec, spec_key, hit);
    if constexpr (PF) take(nr, tk, lane);
    return nx;
  }

  // Every LDS beam position from sz to cap holds kPadKey (above every key):
  // set once per query; merges only write below the new sz, which never
  // shrinks.  The rank search then needs no bounds test.  The rank counts
  // start at zero, and every merge leaves them so.
  __device__ __forceinline__ void pad_beam(int lane) {
#pragma unroll
    for (int k = 0; k < Q; k++)
      if (k * kWave + lane < cap) beam[k * kWave + lane] = kPadKey;
    if constexpr (kCounts) {
#pragma unroll
      for (int k = 0; k < Q; k++) rcount[k * kWave + lane] = 0u;
    }
  }

  // Beam position P from the register copy (kPadKey past it), wave-uniform.
  template <int P>
  __device__ __forceinline__ uint64_t reg_pos() const {
    if constexpr (P < Q * kWave)
      return read_lane_u64(ck[P % Q], P / Q);
    else
      return kPadKey;
  }

  // The 4-ary search's LDS levels of steps S, S / 4, .. 4 (rank_levels).
  template <int S>
  __device__ __forceinline__ void rank_levels(uint32_t& rb, uint32_t top8, uint64_t c0) const {
    if constexpr (S > 1) {
      const uint64_t e1 = lds_u64_min<S - 1>(rb, top8 - 8u * (S - 1));
      const uint64_t e2 = lds_u64_min<2 * S - 1>(rb, top8 - 8u * (2 * S - 1));
      const uint64_t e3 = lds_u64_min<3 * S - 1>(rb, top8 - 8u * (3 * S - 1));
      rb += 8u * (uint32_t)(((e1 < c0 ? 1 : 0) + (e2 < c0 ? 1 : 0) + (e3 < c0 ? 1 : 0)) * S);
      rank_levels<S / 4>(rb, top8, c0);
    }
  }

  // The tail LUT over the pivot table at LDS address 0: entry (m, c) at byte
  // 4096 m + 4 c, inside chunk m's own 4 KB of pivots (pivot (m, c) at
  // 4096 m + 16 c).  Lane l computes codes l, l + 64, l + 128, l + 192 of each
  // chunk; a chunk's 256 pivots are all read before any of its entries is
  // written (the wavefront fence keeps the compiler from moving a write, which
  // never aliases the writing lane's own reads, above another lane's read; the
  // wave's LDS accesses complete in order), and other chunks' bytes are not
  // touched.  An entry is the recompute's own chain (d = q' - p per dimension,
  // acc = d0 d0, then fma in dimension order), so every sum keeps its bits.
  __device__ __forceinline__ void build_tail_lut(int lane) {
    typedef __attribute__((address_space(3))) qv_float4 lds_f4;
    typedef __attribute__((address_space(3))) float lds_f32;
#pragma unroll 1
    for (int m = 0; m < MC; m++) {
      // q' of the chunk's 4 dims: qd[m / 4], lanes 4 (m % 4) .. + 3 (load_query_dpp);
      // the register is selected among values (opaque, so the select does not
      // become an indexed access of qd, which only memory could serve)
      float qr = qd[0];
#pragma unroll
      for (int k = 1; k < kQd; k++) {
        float t = qd[k];
        asm volatile("" : "+v"(t));
        qr = (m >> 2) == k ? t : qr;
      }
      const int l0 = 4 * (m & 3);
      const float q0 = read_lane_f32(qr, l0), q1 = read_lane_f32(qr, l0 + 1);
      const float q2 = read_lane_f32(qr, l0 + 2), q3 = read_lane_f32(qr, l0 + 3);
      lds_f4* const blk4 = (lds_f4*)(uintptr_t)(4096u * (uint32_t)m);
      lds_f32* const blk1 = (lds_f32*)(uintptr_t)(4096u * (uint32_t)m);
      qv_float4 p[4];
#pragma unroll
      for (int j = 0; j < 4; j++) p[j] = blk4[lane + 64 * j];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      float e[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float d0 = q0 - p[j].x, d1 = q1 - p[j].y, d2 = q2 - p[j].z, d3 = q3 - p[j].w;
        float acc = d0 * d0;
        acc = __fmaf_rn(d1, d1, acc);
        acc = __fmaf_rn(d2, d2, acc);
        acc = __fmaf_rn(d3, d3, acc);
        e[j] = acc;
      }
#pragma unroll
      for (int j = 0; j < 4; j++) blk1[lane + 64 * j] = e[j];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }
  }

  __device__ __forceinline__ void enter_tail(int lane) {
    if constexpr (kTail) build_tail_lut(lane);
  }

  // pk from the register copy.
  __device__ __forceinline__ void block_keys() {
#pragma unroll
    for (int j = 0; j < Q - 1; j++) {
      constexpr int kQ = Q;
      const int P = 64 * (j + 1) - 1;
      pk[j] = read_lane_u64(ck[P % kQ], P / kQ);
    }
  }

  // um from the register copy (after a merge reloads it).
  __device__ __forceinline__ void unvisited_mask(int lane) {
    const int nv = sz - lane * Q;
    uint32_t m = 0;
#pragma unroll
    for (int k = 0; k < Q; k++) m |= k < nv && key_unvisited(ck[k]) ? 1u << k : 0u;
    um = m;
  }

  // First unvisited entry of the beam: the first lane L with a bit in um, and
  // its lowest such slot kk, position L Q + kk.  (Q = 1: um is read off the
  // register beam here, whose visited bits are kept current instead.)
  __device__ __forceinline__ void find_unvisited(int lane) {
    if constexpr (Q == 1) unvisited_mask(lane);
    const uint64_t any = __ballot(um != 0);
    if (any) {
      const int L = __ffsll((long long)any) - 1;
      const int kk = __builtin_ctz(read_lane_u32(um, L));
      u = L * Q + kk;
      // its key from the register copy (wave-uniform, so the next node's
      // record address is scalar work), selected among values: opaque, so
      // the select is not turned into one of addresses into ck, an index the
      // compiler can only serve from memory
      uint64_t e = ck[0];
#pragma unroll
      for (int k = 1; k < Q; k++) {
        uint64_t ek = ck[k];
        asm volatile("" : "+v"(ek));
        e = kk == k ? ek : e;
      }
      bu = read_lane_u64(e, L);
    } else {
      u = INT32_MAX;
      bu = ~0ull;
    }
  }

  // Marks the entry at position pos (wave-uniform) visited: in LDS, and in
  // um (bit pos % Q of lane pos / Q).
  __device__ __forceinline__ void mark_visited(int pos, uint64_t key, int lane) {
    if (lane == 0) beam[pos] = key & ~1ull;
    if constexpr (Q == 1) {
      ck[0] &= lane == pos ? ~1ull : ~0ull;
    } else {
      const uint32_t owner = (uint32_t)pos / Q, bit = 1u << ((uint32_t)pos - owner * Q);
      um &= (uint32_t)lane == owner ? ~bit : ~0u;
    }
  }

  // persistent_merge_data's result after persistent_visit_select_dualwarp's
  // compaction and truncation (kernel_helpers.cuh:288-357, 440-472), built by
  // rank.  The reference places a candidate equal to a beam entry (same id,
  // hence same distance) right after it (lower_bound + 1, :300-329) and the
  // adjacent-id compaction then drops it; the min(sz + deg, 2 ef) cap (:350)
  // only removes entries that sit at or beyond ef after compaction, since at
  // most sz <= ef entries are compacted away.  So the new beam is the first ef
  // entries of  beam  U  {candidates whose id is not in the beam}, in key
  // order, and its first unvisited entry is taken and marked visited.
  // has: the lane holds a neighbour.
  //
  // Membership: a neighbour whose id is in the beam has that entry's key
  // (the ADC of one code row against one query is one value), visited bit
  // aside.  So the lower bound r of (c & ~1) in the sorted beam is both
  // the candidate's rank and its membership test: c is in the beam iff
  // beam[r] and c differ only in the visited bit.  Only neighbours below the
  // end of a full beam need it.
  //
  // The selected node only depends on the smallest surviving candidate and
  // the old first unvisited entry, so it is found first and its record is
  // requested (PF) before the rest of the merge, which then overlaps that load,
  // unless it is the first unvisited entry whose record the hop requested at
  // its start (spec).
  // hit: (PF) the selected node is the guessed one (key spec_key), whose
  // record the hop requested at its start.  SEL = false merges without a
  // selection (the first batch of a two-slot hop) and returns -1.
  template <bool SEL, bool PF, bool ROWS = false>
  __device__ __forceinline__ int32_t merge_select(uint64_t nkey, bool has, int lane, Rec& nr, bool spec,
                                                  uint64_t spec_key, bool& hit, CodeRow<MC>* cr = nullptr) {
    const int ef = a.ef;
    // Candidates at or above the last entry of a full beam end beyond ef
    // (lastk: read with the previous merge's register reload).
    const uint64_t last = lastk;
    const bool below = has && nkey < last;
    int r = 0;  // rank in the beam (valid lanes)
    bool valid = below;
    {
      if (__ballot(below)) {
        const uint64_t c0 = nkey & ~1ull;
        uint64_t at;
        if constexpr (kRank8) {
          // cap = 64 Q: r = #{beam entries e : e < c0} by an 8-ary search.
          // Sorted, with kPadKey from sz to cap, the beam puts
          // min(floor(r / 64), Q - 1) of the keys pk below c0, which gives
          // r's 64-entry block at b0 = 64 n0 <= cap - 64 (beam[cap - 1] is
          // kPadKey or, in a full beam of ef = cap, the last key, which a
          // below candidate is under); then 7 keys at steps of 8 inside it
          // and the 8 keys from there (beam[r] among them): every read lies
          // in [b0, b0 + 63], inside the beam, whatever c0.  Two LDS round
          // trips.  Visited bits do not matter: e < c0 ignores them.
          int n0 = 0;
#pragma unroll
          for (int j = 0; j < Q - 1; j++) n0 += pk[j] < c0 ? 1 : 0;
          r = 64 * n0;
          const uint64_t* const blk8 = beam + r;
          int n1 = 0;
#pragma unroll
          for (int j = 1; j < 8; j++) n1 += blk8[8 * j - 1] < c0 ? 1 : 0;
          r += 8 * n1;
          const uint64_t* const last8 = beam + r;
          uint64_t g[8];
#pragma unroll
          for (int j = 0; j < 8; j++) g[j] = last8[j];
          // g[7] is only selected when n == 7; without this the compiler
          // moves its read into that branch, a third dependent round trip.
          asm volatile("" : "+v"(g[7]));
          int n = 0;
#pragma unroll
          for (int j = 0; j < 7; j++) n += g[j] < c0 ? 1 : 0;
          r += n;
          at = g[7];
#pragma unroll
          for (int j = 6; j >= 0; j--) at = n == j ? g[j] : at;
        } else {
          // r = #{beam entries e : e < c0} by a 4-ary search over the
          // LDS beam: sorted, kPadKey from sz to its capacity cap (>= ef), so
          // a read clamped to cap - 1 sees either a key of the beam or kPadKey
          // (a below candidate is under the last key of a full beam, so even a
          // full-capacity beam never lifts r past it).  A level of step s reads
          // r + s - 1, r + 2 s - 1 and r + 3 s - 1 at once (one LDS round trip)
          // and adds s per key below; steps 4^i from kTop cover 4 kTop - 1 >=
          // 64 Q - 1 positions.  The last level (s = 1) also reads r + 3, so
          // beam[r] for the membership test is one of its four keys.
          //
          // The first level (r = 0 in every lane) reads the same three positions
          // for every lane, so it compares against the register beam's copies,
          // read as wave-uniform values: the same keys, or kPadKey past sz where
          // the LDS read would be clamped to cap - 1 -- equal for the
          // comparison, since a below candidate is under the last key of a
          // full beam.  Visited bits do not matter: e < c0 ignores them.
          constexpr int kCap = Q * kWave;
          constexpr int kTop = kCap <= 64 ? 16 : (kCap <= 256 ? 64 : (kCap <= 1024 ? 256 : 1024));
          {
            const uint64_t e1 = reg_pos<kTop - 1>(), e2 = reg_pos<2 * kTop - 1>(), e3 = reg_pos<3 * kTop - 1>();
            r = ((e1 < c0 ? 1 : 0) + (e2 < c0 ? 1 : 0) + (e3 < c0 ? 1 : 0)) * kTop;
          }
          // LDS byte addresses: rb = beam + 8 r, and the read of position
          // min(r + k, cap - 1) at min(rb, top8 - 8 k) + 8 k, the 8 k in the
          // instruction (every beam lies past the LUT or the pivot table, at
          // least 8 KB in, so top8 - 8 k stays above 0 for the LDS levels'
          // k < 3 kTop / 4 <= 768).  The
          // address is wave-uniform: held in a scalar register, opaque, so the
          // bounds are scalar work of each merge rather than vector registers
          // held across the loop.
          uint32_t b0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_addr(beam));
          asm volatile("" : "+s"(b0));
          const uint32_t top8 = b0 + 8u * (uint32_t)(cap - 1);
          uint32_t rb = b0 + 8u * (uint32_t)r;
          rank_levels<kTop / 4>(rb, top8, c0);
          const uint64_t e0 = lds_u64_min<0>(rb, top8);
          const uint64_t e1 = lds_u64_min<1>(rb, top8 - 8u);
          const uint64_t e2 = lds_u64_min<2>(rb, top8 - 16u);
          uint64_t e3 = lds_u64_min<3>(rb, top8 - 24u);
          // e3 is only selected when n == 3; without this the compiler moves its
          // read into that branch, a fourth dependent LDS round trip.
          asm volatile("" : "+v"(e3));
          const int n = (e0 < c0 ? 1 : 0) + (e1 < c0 ? 1 : 0) + (e2 < c0 ? 1 : 0);
          r = (int)((rb - b0) >> 3) + n;
          at = n == 0 ? e0 : (n == 1 ? e1 : (n == 2 ? e2 : e3));
        }
        valid = below && (at >> 1) != (nkey >> 1);
      }
    }
    const uint64_t vm = __ballot(valid);

    int selpos = -1;
    uint64_t selkey = ~0ull;
    if constexpr (!SEL) {
      if (vm == 0) return -1;
    } else {
    if (vm == 0 && u >= sz) return -1;
    // Smallest surviving candidate and its rank in the beam.
    selpos = u;
    selkey = bu;
    if (vm != 0) {
      int at;
      const uint64_t kv0 = wave_min_key(nkey, valid, &at);
      if (kv0 < bu) {
        selpos = read_lane_i32(r, at);
        selkey = kv0;
      }
    }
    if constexpr (PF) {
      // (the key test, not the position: a winning candidate lands at u too)
      hit = spec && selkey == spec_key;
      if (!hit) {
        fetch((int32_t)key_id(selkey), lane, nr);
        // ROWS: the selected node's code rows too, right behind its record
        // (without the table, rows of the codes' first nodes, which only
        // keep every path ending with rows requested after the record)
        if constexpr (ROWS) {
          const int code_bytes = (int)min(a.num_points * a.num_chunks, (int64_t)0x7fffffff);
          adc_load<MC>(*cr, a.nbr_codes != nullptr ? block((int32_t)key_id(selkey)) : buf_at(a.codes, code_bytes),
                       off_blk);
        }
      }
    }
    if (vm == 0) {
      mark_visited(selpos, selkey, lane);
      find_unvisited(lane);
      return (int32_t)key_id(selkey);
    }
    }

    // Each surviving candidate's rank t among the candidates, and the shift
    // sh of every old entry: the number of candidates whose rank is at or
    // below its position.
    int t = 0;
    uint32_t sh[Q];
    if (kCounts && __popcll(vm) > kCountMin) {
      count_shifts(valid, nkey, r, lane, t, sh);
    } else if (kPacked && __popcll(vm) > kPackedMin && ~vm != 0) {
      packed_shifts(vm, valid, nkey, r, lane, t, sh);
    } else {
      // one candidate at a time (few per hop: most neighbours below the
      // beam's end are already in it)
#pragma unroll
      for (int k = 0; k < Q; k++) sh[k] = 0u;
      for (uint64_t rest = vm; rest; rest &= rest - 1) {
        const int l = __ffsll((long long)rest) - 1;
        const uint64_t c = read_lane_u64(nkey, l);
        const int rc = read_lane_i32(r, l);
        t += c < nkey ? 1 : 0;
#pragma unroll
        for (int k = 0; k < Q; k++) sh[k] += lane * Q + k >= rc ? 1u : 0u;
      }
    }

    // Scatter in place; entries pushed to ef or beyond drop out.
#pragma unroll
    for (int k = 0; k < Q; k++) {
      const int pos = lane * Q + k;
      const int g = pos + (int)sh[k];
      const uint64_t e = Q == 1 ? ck[k] : (ck[k] & ~1ull) | ((um >> k) & 1u);
      if (pos < sz && g < ef) beam[g] = g == selpos ? (e & ~1ull) : e;
    }
    const int f = r + t;
    if (valid && f < ef) beam[f] = f == selpos ? (nkey & ~1ull) : nkey;
    sz = min(sz + (int)__popcll(vm), ef);
    // Register copy of the new beam (the wave's LDS accesses complete in
    // order), and its entry at ef - 1 for the next merge, read in the same
    // round trip.
#pragma unroll
    for (int k = 0; k < Q; k++) {
      const int pos = lane * Q + k;
      ck[k] = pos < sz ? beam[pos] : kPadKey;
    }
    lastk = sz >= ef ? beam[ef - 1] : ~0ull;
    if constexpr (kRank8) block_keys();
    if constexpr (Q > 1) unvisited_mask(lane);
    find_unvisited(lane);
    return SEL ? (int32_t)key_id(selkey) : -1;
  }

  // Survivors above which a merge counts them per rank instead of one at a
  // time (kCounts).
  static constexpr int kCountMin = 2;

  // sh and t by counting: rcount[x] = surviving candidates of rank x (LDS
  // adds), replaced by its inclusive prefix over the beam positions (lane l
  // owns positions [l Q, l Q + Q): a running sum over its Q counts, plus the
  // sum of the lanes below).  A candidate of rank r comes after every
  // candidate of a lower rank (a beam entry lies between them) and before
  // every one of a higher rank, so t = prefix(r - 1) plus the candidates of
  // rank r with a smaller key, counted one at a time where a rank holds
  // several.  rcount is zero again on return.
  __device__ __forceinline__ void count_shifts(bool valid, uint64_t nkey, int r, int lane, int& t,
                                               uint32_t (&sh)[Q]) {
    if (valid) __hip_atomic_fetch_add(rcount + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
    uint32_t* const own = rcount + lane * Q;
    uint32_t run = 0;
#pragma unroll
    for (int k = 0; k < Q; k++) {
      run += own[k];
      sh[k] = run;
    }
    const uint32_t lower = wave_excl_sum(run);
#pragma unroll
    for (int k = 0; k < Q; k++) {
      sh[k] += lower;
      own[k] = sh[k];
    }
    // prefix(r) and prefix(r - 1) (at r = 0 the word before the counts, the
    // beam's last, is read and not used)
    const uint32_t* const at = rcount + min(r, cap - 1);
    const uint32_t upto = at[0];
    const uint32_t before = r > 0 ? at[-1] : 0u;
#pragma unroll
    for (int k = 0; k < Q; k++) own[k] = 0u;
    t = (int)before;
    for (uint64_t rest = __ballot(valid && upto - before > 1u); rest; rest &= rest - 1) {
      const int l = __ffsll((long long)rest) - 1;
      const uint64_t c = read_lane_u64(nkey, l);
      t += read_lane_i32(r, l) == r && c < nkey ? 1 : 0;
    }
  }

  // The same in registers (the kernels without the LDS counts, at Q = 4 and
  // 5, where the loop's Q compares per survivor cost the most and one word
  // holds a lane's counts): lane l's counts of surviving candidates per rank, for
  // its positions l Q + k, as 6-bit fields (field k at bit 6 (k % 5) of word
  // k / 5), each survivor adding one to the field of its rank's owner; with
  // at most 63 survivors neither a count nor a prefix leaves its field.
  static constexpr bool kPacked = !kCounts && (Q == 4 || Q == 5);
  static constexpr int kPW = (Q + 4) / 5;
  static constexpr int kPackedMin = 4;

  // sh and t from the packed counts: the prefix over each lane's fields plus
  // the sum of the lanes below gives sh; a candidate of rank r reads the
  // prefix and the count at r from the lane that owns r (ds_bpermute), and
  // t = prefix(r) - count(r), plus the smaller keys of its rank where the
  // count is above one.
  __device__ __forceinline__ void packed_shifts(uint64_t vm, bool valid, uint64_t nkey, int r, int lane, int& t,
                                                uint32_t (&sh)[Q]) {
    uint32_t cw[kPW];
#pragma unroll
    for (int w = 0; w < kPW; w++) cw[w] = 0u;
    for (uint64_t rest = vm; rest; rest &= rest - 1) {
      const int l = __ffsll((long long)rest) - 1;
      const uint32_t rc = (uint32_t)read_lane_i32(r, l);
      const uint32_t owner = rc / Q, f = rc - owner * Q;
      const uint32_t inc = 1u << (6 * (kPW == 1 ? f : f % 5));
#pragma unroll
      for (int w = 0; w < kPW; w++) cw[w] += (uint32_t)lane == owner && (kPW == 1 || f / 5 == (uint32_t)w) ? inc : 0u;
    }
    uint32_t run = 0;
#pragma unroll
    for (int k = 0; k < Q; k++) {
      run += (cw[k / 5] >> (6 * (k % 5))) & 63u;
      sh[k] = run;
    }
    const uint32_t lower = wave_excl_sum(run);
    uint32_t pw[kPW];
#pragma unroll
    for (int w = 0; w < kPW; w++) pw[w] = 0u;
#pragma unroll
    for (int k = 0; k < Q; k++) {
      sh[k] += lower;
      pw[k / 5] |= sh[k] << (6 * (k % 5));
    }
    const uint32_t rr = (uint32_t)min(r, Q * kWave - 1);
    const uint32_t owner = rr / Q, f = rr - owner * Q;
    const int at = (int)(owner << 2);
    uint32_t pv = (uint32_t)__builtin_amdgcn_ds_bpermute(at, (int)pw[0]);
    uint32_t cv = (uint32_t)__builtin_amdgcn_ds_bpermute(at, (int)cw[0]);
    if constexpr (kPW > 1) {
      const uint32_t pv1 = (uint32_t)__builtin_amdgcn_ds_bpermute(at, (int)pw[1]);
      const uint32_t cv1 = (uint32_t)__builtin_amdgcn_ds_bpermute(at, (int)cw[1]);
      pv = f >= 5 ? pv1 : pv;
      cv = f >= 5 ? cv1 : cv;
    }
    const uint32_t sf = 6u * (kPW == 1 ? f : f % 5);
    const uint32_t upto = (pv >> sf) & 63u, here = (cv >> sf) & 63u;
    t = (int)(upto - here);
    for (uint64_t rest = __ballot(valid && here > 1u); rest; rest &= rest - 1) {
      const int l = __ffsll((long long)rest) - 1;
      const uint64_t c = read_lane_u64(nkey, l);
      t += read_lane_i32(r, l) == r && c < nkey ? 1 : 0;
    }
  }

  // persistent_select_next_no_compact (kernel_helpers.cuh:491-518): the first
  // unvisited entry (the beam never exceeds ef here) is taken and marked.
  __device__ __forceinline__ int32_t select_next_no_compact() {
    const int lane = opaque_lane();
    if (u >= sz) return -1;
    const uint64_t sel = bu;
    mark_visited(u, sel, lane);
    find_unvisited(lane);
    return (int32_t)key_id(sel);
  }
};

// gpruning bookkeeping (kernel_q1.cuh:294-315, 524-545).
struct GPrune {
  int no_improve = 0, last_fc = 0;
  float last_top1 = __int_as_float(0x7f800000), last_topk = __int_as_float(0x7f800000);
};

// Orders a query's LDS set-up before its reads: a workgroup barrier when the
// workgroup is the query's one wave, a compiler fence otherwise (a wave's LDS
// accesses complete in order).
template <int SC>
__device__ __forceinline__ void query_sync() {
  if constexpr (SC == 0)
    __syncthreads();
  else
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// The persistent query loop of one wave: smem is its LDS area, piv the
// shared pivots (SC > 0).
template <class T, int Q, int MC, int SC, int NPL, bool WK = false>
__device__ __forceinline__ void run_queries(const SearchArgs& a, char* smem, const float* piv) {
  const int lane = lane_id();

  while (true) {
    // ---- acquire (StreamingDispatch, src/quiver/kernel_core/policies/dispatch.cuh:39-79)
    int32_t qid = -1;
    uint64_t pub = 0;  // the poller's new mirror value, published by the whole wave below
    if (lane == 0) {
      qid = atomicAdd(&a.counters[0], 1);
      if (qid >= a.nq) {
        qid = -1;
      } else if (a.terminate &&
                 __hip_atomic_load(a.terminate, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)) {
        qid = -1;
      } else if (a.feed_count) {
        // Only the wave holding the lowest unadmitted ticket reads the host's
        // feed word; it publishes what it reads in the device mirror lines
        // that every other waiting wave watches (each ticket its own line;
        // addresses from the ticket, never loop-invariant values the compiler
        // would keep in registers through the hops).
        // Thousands of waves reading host memory, or one device word, at once
        // would crowd the fabric the running queries' loads go through.  Every
        // access is relaxed: the queries are in HBM before the launch, so the
        // feed word orders nothing, and an acquire or release at agent or
        // system scope would invalidate or write back the L2 on each poll.
        uint64_t* const mine = a.feed_mirror + (int64_t)(qid & (kFeedLines - 1)) * kFeedStride;
        const uint64_t t0 = wall_ticks();
        for (uint32_t nap = 0;; nap++) {
          const uint64_t mv = __hip_atomic_load(mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const int32_t seen = (uint32_t)(mv >> 32) == a.feed_epoch ? (int32_t)(uint32_t)mv : 0;
          if (qid < seen) break;
          const bool poller = qid == seen;
          if (poller) {
            const int32_t fed = __hip_atomic_load(a.feed_count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (qid < fed) {
              pub = ((uint64_t)a.feed_epoch << 32) | (uint32_t)fed;
              break;
            }
          }
          if ((poller || (nap & 63) == 63) && a.terminate &&
              __hip_atomic_load(a.terminate, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)) {
            qid = -1;
            break;
          }
          if (wall_ticks() - t0 > a.spin_limit_ticks) {
            atomicOr(&a.counters[2], kErrSpinTimeout);
            qid = -1;
            break;
          }
          if (poller)
            __builtin_amdgcn_s_sleep(4);
          else
            __builtin_amdgcn_s_sleep(32);
        }
      }
    }
    qid = read_lane_i32(qid, 0);
    // one mirror line per lane (kFeedLines == kWave), one instruction
    pub = read_lane_u64(pub, 0);
    if (pub != 0)
      __hip_atomic_fetch_max(a.feed_mirror + (int64_t)opaque_lane() * kFeedStride, pub, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    if (qid < 0) break;
    // Later tickets issue first: the last-admitted queries set the end of the
    // launch, the earlier ones have time to spare.
    switch ((int)(((int64_t)qid * 4) / a.nq)) {
      case 0: __builtin_amdgcn_s_setprio(0); break;
      case 1: __builtin_amdgcn_s_setprio(1); break;
      case 2: __builtin_amdgcn_s_setprio(2); break;
      default: __builtin_amdgcn_s_setprio(3); break;
    }
    if (a.t_start && lane == 0) a.t_start[qid] = wall_ticks();

    Query<T, Q, MC, SC, NPL, WK> Qy(a, smem, piv);
    const float* q = a.queries + (int64_t)qid * a.dim;
    // ---- entry node: the nav-graph search on the raw query when a nav graph is
    // loaded (kernel_q1.cuh:148-174, 199-206), else the medoid.
    const int32_t entry = a.nav_data ? nav_entry<T>(q, a.nav_data, a.nav_graph, a.nav_map, a.nav_nodes, a.dim,
                                                    a.nav_max_m, a.nav_start, (int32_t)a.medoid)
                                     : a.medoid;
    // ---- query into LDS: q - mu for the LUT, fl(fl(q - mu) + mu) for the exact
    // distance (pq_device.cuh:18-20, 33-35).
    for (int i = lane; i < a.dim; i += kWave) {
      const float c = query_elem(q, i) - a.centroid[i];
      Qy.qc[i] = c;
      Qy.qu[i] = c + a.centroid[i];
    }
    query_sync<SC>();
    if constexpr (SC == 0) {
      build_lut_lds(Qy.qc, a.pivots_t, a.chunk_off, a.num_chunks, Qy.lut);
      query_sync<SC>();
    }
    load_query_pre(Qy.qu, a.dim, lane, Qy.quv);
    if constexpr (SC > 0) load_query_dpp(Qy.qc, a.dim, lane, Qy.qd);
    // qc and qu may share their LDS with the beam (lds_plan): no beam store
    // may move above these reads.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    Qy.pad_beam(lane);

    GPrune g;
    int step = 0;
    bool stop = false;
    const bool gpr = a.early_exit == QV_EXIT_GPRUNING;
    auto check = [&]() -> bool {
      const float top1 = read_lane_f32(Qy.td, 0);
      const float topk = Qy.kth_dist();
      const int fc = read_lane_i32(Qy.fc, 0);  // equal in every lane; read as uniform
      const bool improved = fc > g.last_fc || top1 < g.last_top1 || topk < g.last_topk;
      if (step < a.warmup) g.no_improve = 0;
      else g.no_improve = improved ? 0 : g.no_improve + 1;
      g.last_fc = fc;
      g.last_top1 = top1;
      g.last_topk = topk;
      return step >= a.warmup && a.patience > 0 && g.no_improve >= a.patience;
    };

    // count_topk_gt_hits (kernel_helpers.cuh:520-535): top-k entries (a
    // repeated id counted each time, -1 padding skipped) found anywhere in the
    // query's ground-truth row, read four ids per lane.
    const bool sr = a.sr_gt != nullptr;
    int sr_at = -1, sr_h = 0;
    auto sr_hits = [&]() -> int {
      const int32_t* row = a.sr_gt + (int64_t)(qid % a.sr_count) * a.sr_width;
      int32_t g[4];
#pragma unroll
      for (int t = 0; t < 4; t++) g[t] = lane + kWave * t < a.sr_width ? row[lane + kWave * t] : -1;
      int hits = 0;
      for (int i = 0; i < a.topk; i++) {
        const int32_t id = Qy.id_at(i);
        if (id < 0) continue;
        hits += __ballot(g[0] == id || g[1] == id || g[2] == id || g[3] == id) != 0 ? 1 : 0;
      }
      return hits;
    };

    auto log_hop = [&](int32_t v) {
      if (a.rec_ids && lane == 0 && step < a.rec_cap) {
        a.rec_ids[(int64_t)qid * a.rec_cap + step] = v;
        a.rec_dists[(int64_t)qid * a.rec_cap + step] = Qy.last_e;
      }
    };

    NodeRec<T, NPL> nr;
    Taken<NPL> tk;
    CodeRow<MC> cr;
    bool have = false;
    // Tail mode probe (kTail): from every 32nd hop on, the wave requests its
    // workgroup's count of ended waves and reads it at its next probe, so the
    // load never stalls a hop.  With every other wave of the workgroup ended
    // it builds its LUT (enter_tail) and returns true, and the search goes on
    // in the loop's tail-mode copy.  A wave ends once its ticket is past nq
    // or the search is terminated (or its feed wait timed out, which fails the
    // search), so this query is then the wave's last as well: the launcher
    // passes wg_done only for workgroups of two waves or more, where that
    // holds.  (The address goes through an opaque lane value so the load is a
    // vector one: a scalar load's wait would also wait for the LDS traffic.
    // Also reading the ticket counter here measured up to a fifth slower.)
    constexpr bool kTail = Query<T, Q, MC, SC, NPL>::kTail;
    int32_t probe_w = 0, probe_at = 32;
    bool probing = false;
    auto tail_probe = [&]() -> bool {
      if constexpr (kTail) {
        if (!a.wg_done) return false;
        if (probing) {
          probing = false;
          if (read_lane_i32(probe_w, 0) >= (int)(blockDim.x / kWave) - 1) {
            Qy.enter_tail(lane);
            if (lane == 0) atomicAdd(&a.counters[4], 1);
            return true;
          }
        } else if (step >= probe_at) {
          const int z = opaque_lane() >> 8;  // 0
          probe_w = __hip_atomic_load(a.wg_done + blockIdx.x + z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          probing = true;
          probe_at = step + 32;
        }
      }
      return false;
    };
    // Expansion for the pipe lanes: nxt is the expansion expected next (-1:
    // not known), whose record (and rows) the hop requests once it has read
    // v's; pf is the node so requested, fetched again when the guess was wrong.
    int32_t pf = -1;
    auto expand = [&](int32_t v, int32_t nxt, auto tl) -> int32_t {
      if (v != pf) {
        Qy.fetch(v, lane, nr);
        Qy.take(nr, tk, lane);
        have = false;
      }
      const int32_t nx = Qy.template hop<2, decltype(tl)::value>(v, tk, nr, cr, have, nxt);
      pf = NPL == 1 ? nxt : -1;
      return nx;
    };

    if (a.pipe_w == 1) {
      // One pipe lane (kernel_q1.cuh:199-397 boot, then 407-670): the node a
      // hop selects is the next one expanded, so its record is requested while
      // the hop finishes.
      Qy.fetch(entry, lane, nr);
      Qy.take(nr, tk, lane);
      int32_t v = entry;
      // true: go on from v in tail mode
      auto w1_loop = [&](auto tl) -> bool {
        constexpr bool TL = decltype(tl)::value;
        while (true) {
          const int32_t nx = Qy.template hop<1, TL>(v, tk, nr, cr, have);
          log_hop(v);
          ++step;
          bool to_tail = false;
          if constexpr (!TL) to_tail = tail_probe();
          if (gpr && check()) {
            stop = true;
            return false;
          }
          // per-step recall, after the early-exit test (kernel_q1.cuh:354-364)
          if (sr) {
            const int h = sr_hits();
            if (h >= a.sr_required) {
              sr_at = step;
              sr_h = h;
              stop = true;
              return false;
            }
          }
          if (nx < 0) return false;
          v = nx;
          if (to_tail) return true;
        }
      };
      if (w1_loop(BoolC<false>{})) {
        if constexpr (kTail) w1_loop(BoolC<true>{});
      }
      goto finish;
    }
    {
    // ---- boot (kernel_q1.cuh:199-397)
    int32_t first = expand(entry, -1, BoolC<false>{});
    log_hop(entry);
    step = 1;
    if (gpr && check()) {
      stop = true;
      first = -1;
    }
    // Lane w < W of pipe_node holds the node of pipe lane w (-1: idle).  The
    // pipe state stays in registers: no LDS round trip and no barrier, whose
    // memory fence would also wait for the record requested by the last hop.
    const int W = a.pipe_w;
    int32_t pipe_node = lane == 0 ? first : -1;
    for (int w = 1; w < W; w++) {
      const int32_t nx = Qy.select_next_no_compact();
      pipe_node = lane == w ? nx : pipe_node;
    }
    uint32_t ready = stop ? 0u : (uint32_t)__ballot(lane < W && pipe_node != -1);

    // ---- pipe loop, every issued lane served at once (kernel_q1.cuh:407-670);
    // tail mode is entered between rounds.  true: go on in tail mode
    auto pipe_loop = [&](auto tl) -> bool {
    while (!stop && ready) {
      const uint32_t cur = ready;
      for (int w = 0; w < W; w++) {
        if (!(cur & (1u << w))) continue;
        const int32_t v = read_lane_i32(pipe_node, w);
        // expected next: the round's next issued lane, else the node this
        // round gave its first lane (the next round starts there unless an
        // idle lane below it is refilled)
        const uint32_t later = cur & ~((2u << w) - 1u);
        const int f = __builtin_ctz(cur);
        const int32_t nxt = later ? read_lane_i32(pipe_node, __builtin_ctz(later))
                                  : (f == w ? -1 : read_lane_i32(pipe_node, f));
        int32_t nx = expand(v, nxt, tl);
        log_hop(v);
        ++step;
        if (gpr && check()) {
          stop = true;
          nx = -1;
        }
        pipe_node = lane == w ? nx : pipe_node;
      }
      if (stop) break;
      for (int w = 0; w < W; w++) {
        if (cur & (1u << w)) continue;
        const int32_t nx = Qy.select_next_no_compact();
        pipe_node = lane == w ? nx : pipe_node;
      }
      ready = (uint32_t)__ballot(lane < W && pipe_node != -1);
      if constexpr (!decltype(tl)::value) {
        if (ready && tail_probe()) return true;
      }
    }
    return false;
    };
    if (pipe_loop(BoolC<false>{})) {
      if constexpr (kTail) pipe_loop(BoolC<true>{});
    }
    }

  finish:
    // ---- finish (kernel_q1.cuh:662-704)
    if (sr) {
      if (sr_at < 0) sr_h = sr_hits();
      if (lane == 0) {
        a.sr_step[qid] = sr_at;
        a.sr_hits[qid] = sr_h;
      }
    }
    if (lane < a.topk) {
      a.out_ids[(int64_t)qid * a.topk + lane] = Qy.ti;
      a.out_dists[(int64_t)qid * a.topk + lane] = Qy.td;
    }
    if constexpr (WK) Qy.write_wide(qid, lane);
    if (lane == 0) {
      if (a.out_found) a.out_found[qid] = Qy.fc;
      if (a.out_hops) a.out_hops[qid] = step;
      if (a.out_stopped) a.out_stopped[qid] = stop ? 1 : 0;
      if (a.out_evals) a.out_evals[qid] = Qy.evals;
      if (a.t_end) a.t_end[qid] = wall_ticks();
      atomicAdd(&a.counters[1], 1);
      if (a.ring) {
        // relaxed: the host takes the entry as the query's completion time
        // only; it reads the results once the launch has ended
        const int32_t pos = atomicAdd(&a.counters[3], 1);
        __hip_atomic_store(&a.ring[pos], qid + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
    }
    query_sync<SC>();
  }
  // This wave has no more queries: one more ended wave of its workgroup (the
  // tail-mode probe of the others reads it).  Release at workgroup scope: the
  // count is published after this wave's last pivot reads are done.
  if constexpr (Query<T, Q, MC, SC, NPL>::kTail) {
    if (a.wg_done && lane == 0)
      __hip_atomic_fetch_add(a.wg_done + blockIdx.x, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// One query per workgroup of one wave, its LUT in LDS.  WK: top-k above 64
// (entries past the 64th in LDS after the query's area).
template <class T, int Q, int MC, int NPL, bool WK = false>
__global__ __launch_bounds__(64) void search_kernel(SearchArgs a) {
  extern __shared__ __align__(16) char smem[];
  run_queries<T, Q, MC, 0, NPL, WK>(a, smem, nullptr);
}

// One workgroup per CU, one query per wave: the workgroup holds the pivots
// once and every wave recomputes the LUT entries it needs (chunks of SC
// dimensions), so the CU's LDS serves more queries than with a 32 KB LUT per
// query.  Beams of more than 7 positions per lane (ef > 448; their LDS beams
// allow 3 to 7 queries per CU) and two neighbour slots per lane (two code
// rows per lane in flight) take 8 waves at most, which leaves each wave up to
// 256 registers.
template <class T, int Q, int MC, int SC, int NPL>
__global__ __launch_bounds__(kWave * sp_max_waves(Q, NPL)) void search_kernel_sp(SearchArgs a) {
  extern __shared__ __align__(16) char smem[];
  float* piv = reinterpret_cast<float*>(smem);
  // pivots_t is [dim][256]; dim i of code c goes where adc_recompute reads it
  for (int idx = threadIdx.x; idx < a.dim * kPivots; idx += blockDim.x) {
    const int i = idx >> 8, c = idx & (kPivots - 1);
    piv[piv_index<SC>(i, c)] = a.pivots_t[idx];
  }
  __syncthreads();
  const int w = threadIdx.x / kWave;
  const LdsPlan pl = lds_plan(a.num_chunks, a.dim, Q, false, a.ef, a.topk);
  run_queries<T, Q, MC, SC, NPL>(a, smem + piv_bytes(a.dim) + w * pl.total, piv);
}

}  // namespace
