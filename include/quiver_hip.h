/*
 * quiver_hip.h -- C ABI of the MI355X-native Quiver query path.
 *
 * Plain pointers and sizes only.  Every call returns a QV_* status; on failure
 * qv_last_error() returns a thread-local message.  Nothing here throws or exits.
 * Host buffers are owned by the caller and are never registered with the HIP
 * runtime; device state (graph pages, PQ codes, tables, search scratch) is owned
 * by the library and freed by qv_index_close().  One search may run per index
 * handle at a time; calls are blocking.
 *
 * Each entry point names the reference interface it replaces
 * (ruc-system/quiver-ae paths).
 */
#ifndef QUIVER_HIP_H
#define QUIVER_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QV_OK 0
#define QV_EINVAL -1      /* bad argument or option */
#define QV_EIO -2         /* file missing, short or malformed */
#define QV_EHIP -3        /* HIP runtime error */
#define QV_ETIMEDOUT -4   /* search exceeded qv_search_opts.timeout_s */
#define QV_EUNSUPPORTED -5/* feature this library does not implement (SPDK, R > 128, ...) */
#define QV_ENOMEM -6      /* host or device allocation failed */
#define QV_EINDEX -7      /* index content invalid (ids out of range, ...) */

/* Element types: shared::DataType (src/shared/common/data_type.hpp:5-9). */
#define QV_UINT8 0
#define QV_FLOAT 1
#define QV_INT8 2

/* Early-exit policies: quiver::EarlyExitPolicy (src/quiver/io_control.cuh:41-46)
 * as exposed by the CLI (bin/quiver_search.cu:48-54). */
#define QV_EXIT_NONE 0
#define QV_EXIT_GPRUNING 2

/* Admission modes of qv_search. */
#define QV_ADMIT_STREAMING 0 /* window of num_blocks*Q + prefeed queries, as
                                run_persistent_search (src/quiver/search.cu:827-1051) */
#define QV_ADMIT_BATCH 1     /* every query admitted when the clock starts */
#define QV_ADMIT_STATIC 2    /* sequential batches of num_blocks*Q queries, each
                                admitted when the previous one has completed;
                                a query's latency is its batch's wall time, as
                                run_static_batch_search (src/quiver/search.cuh:
                                68-95, search.cu:1703-1796) */

/* Search kernel variants (no counterpart in the reference, whose one kernel
 * keeps a per-query LUT in shared memory).  Both give identical results. */
#define QV_KERNEL_AUTO 0          /* per-query LUT while its resident slots hold every
                                     query the call can have in flight (min(nq,
                                     num_blocks x queries_per_block)), else shared
                                     pivots where the index allows them */
#define QV_KERNEL_LUT 1           /* per-query fp32 LUT in LDS, one wave per workgroup */
#define QV_KERNEL_SHARED_PIVOTS 2 /* PQ pivots once per CU in LDS, each LUT entry
                                     recomputed where it is read; needs chunks of
                                     4 dims (M = 32) or 2 dims (M = 48) */

typedef struct qv_index qv_index;

/* shared::Layout (src/shared/common/layout.hpp:7-19) plus the PQ shape. */
typedef struct {
  int64_t num_data;
  int64_t num_dims;
  int64_t max_m0;         /* R */
  int64_t enter_point;    /* medoid */
  int64_t data_size;
  int64_t node_size;
  int64_t num_pages;
  int64_t nodes_per_page;
  int32_t data_type;      /* QV_UINT8 / QV_FLOAT / QV_INT8 */
  int32_t num_chunks;     /* PQ M */
  int32_t device;
  int32_t slots_per_cu;   /* concurrent queries (waves) per CU of the kernel a full
                             batch takes at ef <= 64 */
  int64_t device_bytes;   /* HBM held by the index */
  int64_t nav_nodes;      /* nodes of the loaded nav graph (0: none, entry = medoid) */
  int32_t nav_max_m;      /* its max degree */
  int32_t reserved;
} qv_index_info;

/* Replaces bin_common::prepare_search_setup (bin/common/search_setup.hpp:73-119):
 * find_index_file / find_pq_prefix discovery (bin/common/index_discovery.hpp:57-103),
 * parse_diskann_metadata (bin/common/metadata.hpp:15-72), PQSearch::read_data
 * (src/shared/index/pq_search.cu:62-114), create_mem_loader_sync heap mode
 * (src/shared/io/mem_loader.cpp:28-44) and PQSearch::init_device
 * (src/shared/index/pq_search.cu:116-177).  The page image, the codes and the PQ
 * tables are placed in HBM of `device`.  memory_backend "heap" reads the page
 * image with stdio (mem_loader.cpp:28-44), "mmap" maps the file read-only and
 * checks its size as mem_loader.cpp:46-85 does; both copy it once, at open.
 * memory_index_file may be NULL (defaults to the discovered index file, as
 * --memory-index-file does). */
int qv_index_open(const char* index_dir, const char* data_type,
                  const char* memory_backend, const char* memory_index_file,
                  int device, qv_index** out);

/* A handle from an index the caller already holds in host memory -- what
 * quiver::run_persistent_search (src/quiver/search.cuh:45-66) receives from
 * its caller instead of file names: the shared::Layout (layout.hpp:7-19; of
 * `layout` the fields num_data, num_dims, max_m0, enter_point, data_size,
 * node_size, num_pages, nodes_per_page and data_type are read), the page
 * image of its IndexLoader (num_pages x 4096 bytes, page k = page k + 1 of the
 * disk index, as MemLoaderSync::load_heap holds it, mem_loader.cpp:28-44, and
 * as submit_direct hands pages out, :104-117) and the host tables of its
 * PQSearch (PQSearchData, pq_search.hpp:13-29: centroid [dim], pivots
 * [256][dim], chunk_id [dim] non-decreasing -- chunks are contiguous
 * dimension ranges -- and compressed_data [num_data][num_chunks]).  The same
 * checks as qv_index_open; everything is copied to HBM of `device`, nothing of
 * the caller's is kept. */
int qv_index_from_memory(const qv_index_info* layout, const uint8_t* pages,
                         const float* centroid, const float* pivots,
                         const int32_t* chunk_id, int32_t num_chunks,
                         const uint8_t* codes, int device, qv_index** out);

/* Sets (or replaces) the navigation graph of a handle from the host arrays of
 * a shared::NavGraph (nav_graph.hpp): data [num_node][dim] elements of the
 * index type, graph [num_node][max_m] (-1 after a node's neighbours), mapping
 * [num_node] base ids, start; max_m <= 32 (nav_graph.cu:58). */
int qv_index_set_nav(qv_index* index, const void* data, const int32_t* graph,
                     const int32_t* mapping, int64_t num_node, int32_t max_m,
                     int32_t start);

/* Where the page image (vectors + adjacency, the bulk of an index) lives. */
#define QV_GRAPH_HBM 0  /* device memory (default) */
#define QV_GRAPH_HOST 1 /* pinned host memory the kernel reads over the host link,
                           for indexes larger than HBM; codes, tables and search
                           state stay in HBM.  The reference's own placement: its
                           memory backend keeps the graph in host memory and its
                           loader copies pages into GPU-visible buffers
                           (mem_loader.cpp:98-117). */

/* qv_index_open with an explicit page-image placement (QV_GRAPH_*). */
int qv_index_open_ex(const char* index_dir, const char* data_type,
                     const char* memory_backend, const char* memory_index_file,
                     int device, int32_t graph_placement, qv_index** out);

/* Moves the page image of an open handle (QV_GRAPH_HBM <-> QV_GRAPH_HOST),
 * e.g. to serve a GPU-built index from host memory.  No reference counterpart:
 * the reference fixes the placement by its loader choice at startup. */
int qv_index_place_graph(qv_index* index, int32_t graph_placement);

int qv_index_get_info(const qv_index* index, qv_index_info* out);

/* Loads (or replaces) the navigation graph of a handle from nav_dir
 * (nav_index, nav_index.data, map.txt; NavGraph::init, src/shared/index/
 * nav_graph.cu:12-73).  qv_index_open loads one by itself when index_dir holds
 * nav_index or nav/nav_index (find_nav_dir, bin/common/index_discovery.hpp:
 * 105-115).  With a nav graph every query starts from the node the in-kernel
 * nav search returns (inkernel_nav_entry, src/quiver/kernel_core/
 * inkernel_nav.cuh:61-200) instead of the medoid. */
int qv_index_load_nav(qv_index* index, const char* nav_dir);

/* Builds (enable != 0) or frees the handle's neighbour code table: for every
 * node v, the PQ code rows of its max_m neighbour slots stored contiguously
 * ([num_data][max_m][num_chunks] bytes in HBM, zero past v's degree; 20.5 GB
 * at 10M points with R = 64, M = 32).  No counterpart in the reference: it is
 * a second layout of the codes the reference reads row by row
 * (kernel_helpers.cuh:271-287).  With it a hop reads its node's rows as one
 * block whose address needs no neighbour ids, so the next node's rows are
 * requested together with its record; results are unchanged.  Needs
 * num_chunks 32 or 48 (the chunk counts whose hop reads the table) and
 * max_m <= 64 (QV_EUNSUPPORTED otherwise); QV_ENOMEM when the device lacks
 * the room (plus 1 GiB). */
int qv_index_neighbour_codes(qv_index* index, int32_t enable);

/* ---- Host-only pieces of the setup path (no GPU needed) ---------------------
 * qv_find_index_files: find_index_file + find_pq_prefix
 * (bin/common/index_discovery.hpp:57-103); writes NUL-terminated paths.
 * qv_read_layout: parse_diskann_metadata (bin/common/metadata.hpp:15-72);
 * fills the layout fields of `out` (PQ and device fields are zero).
 * qv_read_index_pages: the heap memory backend's image
 * (MemLoaderSync::load_heap, src/shared/io/mem_loader.cpp:28-44): page k of
 * dst is page k+1 of the file, for k < num_pages. */
int qv_find_index_files(const char* index_dir, char* index_file, char* pq_prefix,
                        int32_t capacity);
int qv_read_layout(const char* index_file, const char* data_type, qv_index_info* out);
int qv_read_index_pages(const char* index_file, int64_t num_pages, uint8_t* dst);

/* Frees every device and host resource of the handle.  NULL is accepted. */
void qv_index_close(qv_index* index);

/* Options of run_persistent_search (src/quiver/search.cuh:45-66) and of the
 * quiver_search CLI (bin/quiver_search.cu:61-147). */
typedef struct {
  int32_t num_blocks;        /* --num-blocks; 0 fills the GPU */
  int32_t queries_per_block; /* --queries-per-block, 1..8: num_blocks x this many query
                                slots (search.cu:393-399), one wave each; the launch
                                stops at the device's resident capacity */
  int32_t pipe_width;        /* --pipe-width, 1..16 */
  int32_t early_exit;        /* QV_EXIT_NONE / QV_EXIT_GPRUNING */
  int32_t gpruning_warmup;   /* 10 in the reference CLI */
  int32_t gpruning_patience; /* 8 in the reference CLI */
  int32_t prefeed;           /* QUIVER_PREFEED */
  int32_t admit_min_batch;   /* QUIVER_ADMIT_MIN_BATCH */
  int32_t admission;         /* QV_ADMIT_STREAMING / QV_ADMIT_BATCH */
  int32_t device_buffers;    /* 1: queries and outputs are device pointers */
  double timeout_s;          /* 0: no limit */
  int32_t skip_nav;          /* --skip-nav: medoid entry even with a nav graph loaded */
  int32_t kernel;            /* QV_KERNEL_AUTO / QV_KERNEL_LUT / QV_KERNEL_SHARED_PIVOTS */
  /* Per-step recall (--per-step-recall; PerStepRecallOptions, src/quiver/
   * search.cuh:17-28, applied as kernel_q1.cuh:354-364, 662-667): when
   * step_recall_gt is not NULL, query i stops after the first step at which
   * ceil(threshold x topk) of its top-k ids appear in ground-truth row
   * i % count.  Host memory, also with device_buffers: gt [count][width]
   * int32 (width 1..256, >= topk), outputs step [nq] (-1 if never reached) and
   * hits [nq] (may be NULL).  Pipe width 1 and queries_per_block 1 only, as
   * in the reference (search.cu:492-505). */
  const int32_t* step_recall_gt;
  int32_t step_recall_gt_width;
  int32_t step_recall_gt_count;
  float step_recall_threshold;  /* (0, 1]; --recall-threshold, 0.9 by default */
  int32_t* step_recall_step;
  int32_t* step_recall_hits;
  /* Open-loop arrival (streaming admission only; no counterpart in the
   * reference, whose admission loop refills a window as queries complete,
   * search.cu:983-1051): with arrival_qps > 0, queries arrive in groups of
   * arrival_batch at a fixed rate, group j at t0 + j * arrival_batch /
   * arrival_qps, and each group is admitted on its clock however many queries
   * are still in flight.  A query's latency runs from its group's scheduled
   * arrival.  0 (default): the reference's closed window. */
  double arrival_qps;
  int32_t arrival_batch;     /* queries per arrival, >= 1 (default 1) */
  int32_t reserved0;
} qv_search_opts;

/* shared::RunReport (src/shared/common/run_report.hpp:32-56) for one search. */
typedef struct {
  double qps;
  double search_time_s;      /* first admission -> results ready */
  double lat_avg_ms, lat_p50_ms, lat_p90_ms, lat_p99_ms, lat_p999_ms, lat_max_ms;
  double avg_hops;           /* expanded nodes per query (finish step) */
  double kernel_ms;          /* search kernel duration from HIP events */
  int32_t num_blocks;        /* workgroups launched (= concurrent query slots) */
  int32_t max_inflight;      /* admission window: slots + prefeed */
  int32_t early_stopped;     /* queries ended by gpruning */
  int32_t kernel;            /* the search kernel that ran: QV_KERNEL_LUT or QV_KERNEL_SHARED_PIVOTS */
  double total_hops;         /* expanded nodes over all queries */
  double total_evals;        /* neighbour ADC evaluations over all queries */
  int32_t tail_queries;      /* queries finished in tail mode (shared pivots: the
                                workgroup's last wave, the pivot table turned
                                into its own LUT); no reference counterpart */
  int32_t reserved1;
} qv_search_report;

void qv_search_opts_default(qv_search_opts* opts);

/* Replaces quiver::run_persistent_search (src/quiver/search.cuh:45-66).
 * queries: [nq][dim] float (uint8/int8 queries are passed as floats, as
 * load_queries_as_float does, bin/common/data_io.hpp:73-108).
 * ids [nq][topk] int32 (-1 padded), dists [nq][topk] float (+inf padded),
 * found [nq] int32 (may be NULL), report may be NULL.
 * topk in [1, 1024], ef_search in [1, 2048]; with topk above 64 or ef_search
 * above 1024 the search runs on the per-query-LUT kernel (a forced
 * QV_KERNEL_SHARED_PIVOTS is QV_EUNSUPPORTED there), which keeps top-k entries
 * past the 64th in LDS.
 * With opts->device_buffers, queries/ids/dists/found are device pointers. */
int qv_search(qv_index* index, const float* queries, int64_t nq, int32_t dim,
              int32_t topk, int32_t ef_search, const qv_search_opts* opts,
              int32_t* ids, float* dists, int32_t* found, qv_search_report* report);

/* No counterpart in the reference.  For callers that cannot allocate (tight
 * serving loops, harnesses that forbid hipMalloc): qv_search with every query
 * admitted at launch, all of d_queries / d_ids / d_dists / d_found (may be
 * NULL) device pointers, and the search's scratch (dispatch counters,
 * per-query hop, evaluation and early-exit counts, the shared-pivot kernel's
 * count of ended waves per workgroup) taken from one fixed device array of
 * QV_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends.  It calls no hipMalloc, hipHostMalloc, hipFree or memset of any kind.
 * It is synchronous: it runs on the handle's own stream and returns once the
 * results are in the caller's device buffers, so it cannot be captured into
 * a caller's HIP graph.  Limits: 1..QV_NOALLOC_MAX_QUERIES queries per call
 * (QV_EINVAL beyond); opts->timeout_s must be 0 (no deadline); no per-step
 * recall or open-loop arrival.  Results (ids, distances, found counts, hop
 * and evaluation totals, early exits) equal qv_search's.  All calls on one
 * GPU share its array and are serialised by a lock per GPU; calls on
 * different GPUs run independently.  The report has no latency percentiles
 * (queries are not stamped). */
#define QV_NOALLOC_SCRATCH_BYTES (12 * 1024 * 1024 + 256 + 16 * 1024)
#define QV_NOALLOC_MAX_QUERIES (1024 * 1024)
int qv_search_noalloc(qv_index* index, const float* d_queries, int64_t nq, int32_t dim,
                      int32_t topk, int32_t ef_search, const qv_search_opts* opts,
                      int32_t* d_ids, float* d_dists, int32_t* d_found,
                      qv_search_report* report);

/* Per-query hop counts of the last qv_search on this handle, [nq] int32. */
int qv_last_hops(const qv_index* index, int32_t* hops, int64_t nq);

/* Per-query latencies (ms) of the last qv_search on this handle, [nq] double,
 * in query order: completion observed by the host minus admission (streaming
 * admission), or completion minus the first query's start on the device clock
 * (batch admission) -- the figures qv_search_report's percentiles summarise
 * (src/quiver/search.cu:1006-1024). */
int qv_last_latencies(const qv_index* index, double* ms, int64_t nq);

/* Thread-local message of the last failing call on this thread. */
const char* qv_last_error(void);

/* Device count and gfx name of `device` (for diagnostics). */
int qv_device_info(int device, char* name, int32_t name_len, int32_t* num_cus,
                   int64_t* total_mem);

/* ---- Device-buffer plumbing (no reference counterpart) ---------------------
 * For callers that reach the library through a plain FFI (ctypes) and have no
 * HIP binding of their own: allocate, copy and clear device memory on the
 * library's HIP runtime.  kind: 0 host->device, 1 device->host, 2 device->device
 * (one GPU, 16-byte aligned: a grid-stride copy kernel, else hipMemcpy). */
int qv_device_count(int32_t* count);
/* Free and total device memory of `device` (hipMemGetInfo). */
int qv_device_mem_info(int device, int64_t* free_bytes, int64_t* total_bytes);
int qv_dev_alloc(int device, int64_t bytes, void** out);
int qv_dev_free(void* ptr);
int qv_dev_copy(void* dst, const void* src, int64_t bytes, int32_t kind);
int qv_dev_clear(void* ptr, int64_t bytes);

/* ---- PQ look-up tables (src/shared/index/pq_device.cuh:9-36) ----------------
 * Builds LUT[q][m][256] for nq queries on the device.  Tables may come from an
 * index (qv_lut_build) or be passed raw (qv_lut_build_raw: centroid [dim],
 * pivots_t [dim][256], chunk_offsets [M+1], all device pointers, as are queries,
 * luts and q_used).  q_used ([nq][dim], may be NULL) receives fl(fl(q-mu)+mu). */
int qv_lut_build(qv_index* index, const float* d_queries, int64_t nq,
                 float* d_luts, float* d_q_used);
int qv_lut_build_raw(const float* d_centroid, const float* d_pivots_t,
                     const int32_t* d_chunk_offsets, int32_t dim, int32_t num_chunks,
                     const float* d_queries, int64_t nq, float* d_luts,
                     float* d_q_used, int device);

/* ---- ADC gather-sum + top-k microbenchmark ---------------------------------
 * The fused ADC of persistent_merge_data (src/quiver/kernel_core/
 * kernel_helpers.cuh:271-287) with top-k maintenance, in isolation:
 * for each query q and s in [0, ids_per_query): d = sum_m LUT[q][m][codes[id][m]]
 * (sequential fp32 sum over m) with id = ids[q][s]; keeps the topk smallest
 * under (d, s), i.e. the reference's first-found-wins insert applied in s order.
 * All pointers are device pointers: luts [nq][M][256] f32, codes
 * [num_codes][M] u8, ids [nq][ids_per_query] int32 (each in [0, num_codes);
 * the base address 16-byte aligned, else QV_EINVAL; an id outside the range
 * reads a row inside the table and its distance is unspecified),
 * out_ids [nq][topk] int32, out_dists [nq][topk] f32, dist_sums [nq] f64 (may
 * be NULL; the sum of all distances of a query).  elapsed_ms (may be NULL)
 * receives the kernel time from HIP events. */
int qv_adc_bench(const float* d_luts, int32_t num_chunks, const uint8_t* d_codes,
                 int64_t num_codes, const int32_t* d_ids, int64_t nq,
                 int64_t ids_per_query, int32_t topk, int32_t* d_out_ids,
                 float* d_out_dists, double* d_dist_sums, int device,
                 float* elapsed_ms);

/* Random row gather alone (no reference counterpart; a measurement aid): reads
 * the 32-byte rows d_rows[d_ids[i]] for i < n exactly as qv_adc_bench fetches
 * code rows (lane pairs, one 32-byte access per row) and XOR-folds them into
 * d_fold[ceil(2 n / 256)] (one word per 256-thread workgroup).  Ids are clamped
 * into [0, num_rows).  Its rows per second bound the ADC gather from above on
 * the device at hand.  elapsed_ms (may be NULL) receives the kernel time. */
int qv_gather_bench(const uint8_t* d_rows, int64_t num_rows, const int32_t* d_ids,
                    int64_t n, uint32_t* d_fold, int device, float* elapsed_ms);

/* The gather for rows of row_bytes (32, 64, 128 or 256) over one table of
 * table_bytes (16-byte aligned): row i is d_table + (d_ids[i] >> id_shift) *
 * row_bytes, clamped into the table; XOR-folded into d_fold[ceil(n *
 * row_bytes / 16 / 256)].  With one id array and shifts 0, 1, 2, 3 the same
 * number of uniformly random rows of 32 to 256 bytes are read from the same
 * table, which tells a per-row cost from a per-byte one (no reference
 * counterpart; a measurement aid).  elapsed_ms (may be NULL) receives the
 * kernel time. */
int qv_gather_rows_bench(const uint8_t* d_table, int64_t table_bytes, int32_t row_bytes,
                         const int32_t* d_ids, int64_t n, int32_t id_shift, uint32_t* d_fold,
                         int device, float* elapsed_ms);

/* The random row gather in a configurable shape, for the access-rate matrix
 * (no reference counterpart; a measurement aid): rows of row_bytes (32, 64,
 * 128 or 256) from a table of table_rows rows, row i = (d_ids[i] * row_mul)
 * >> 32 with row_mul = floor(table_rows * 2^32 / id_range), clamped to the
 * last row (ids uniform over [0, id_range) land uniformly in the table;
 * table_rows < 2^32, id_range <= 2^32); rows_in_flight (1, 2 or 4) rows
 * requested per group of row_bytes / 16 lanes before any is used;
 * waves_per_cu (8, 16 or 32) resident waves per CU (a persistent grid sized
 * through its LDS); nontemporal != 0 for nontemporal loads.  The XOR of every
 * 32-bit word read goes into d_fold[0] (XORed in: clear it first).
 * elapsed_ms and waves_launched (may be NULL) receive the kernel time and the
 * waves launched. */
int qv_gather_sweep_bench(const uint8_t* d_table, int64_t table_rows, int32_t row_bytes,
                          const int32_t* d_ids, int64_t n, int64_t id_range,
                          int32_t rows_in_flight, int32_t waves_per_cu, int32_t nontemporal,
                          uint32_t* d_fold, int device, float* elapsed_ms,
                          int32_t* waves_launched);

/* Sequential read of nbytes (a multiple of 16, 16-byte aligned) from d_src,
 * XOR-folded into d_fold[min(QV_STREAM_READ_BLOCKS, ceil(nbytes / 4096))] (no
 * reference counterpart; a measurement aid): the device's streaming read
 * bandwidth, reported beside the nominal HBM peak.  elapsed_ms (may be NULL)
 * receives the kernel time. */
#define QV_STREAM_READ_BLOCKS 4096
int qv_stream_read_bench(const uint8_t* d_src, int64_t nbytes, uint32_t* d_fold, int device,
                         float* elapsed_ms);

/* Counter-based fills for synthetic tables: 8-byte word w of the buffer is a
 * function of (seed, w) only; id i is uniform in [0, num_codes) and a function
 * of (seed, i) only. */
int qv_fill_uniform_bytes(uint8_t* d_dst, int64_t nbytes, uint64_t seed, int device);
int qv_fill_uniform_ids(int32_t* d_dst, int64_t count, int64_t num_codes,
                        uint64_t seed, int device);

/* ---- Index construction (DiskANN's build_disk_index is absent: this replaces
 * the build step the reference delegates to deps/DiskANN, CMakeLists.txt:35-39).
 * Writes <out_prefix>_disk.index, <out_prefix>_pq_pivots.bin and
 * <out_prefix>_pq_compressed.bin in the formats the reference reads
 * (bin/common/metadata.hpp:15-72, src/shared/index/pq_search.cu:62-114).
 * base: host [n][dim] of data_type.  CPU build with OpenMP (`threads`, <=0 all). */
typedef struct {
  int32_t R;             /* max degree */
  int32_t L;             /* build beam width */
  float alpha;           /* RobustPrune alpha */
  int32_t num_chunks;    /* PQ M */
  int32_t kmeans_iters;  /* PQ k-means iterations */
  int32_t pq_train_max;  /* training sample size for PQ */
  uint64_t seed;
  int32_t threads;
  int32_t passes;        /* 1: alpha only; 2: 1.0 then alpha */
} qv_build_params;

void qv_build_params_default(qv_build_params* p);

int qv_build_index_cpu(const void* base, int32_t data_type, int64_t n, int32_t dim,
                       const qv_build_params* params, const char* out_prefix);

/* Navigation graph for the per-query entry search (the files NavGraph::init
 * reads, src/shared/index/nav_graph.cu:12-73; the reference ships no builder
 * for them): a Vamana graph of degree params->R <= 32 (default 28, the number
 * of neighbours the nav search reads per node) over host rows [num_rows][dim]
 * whose base ids are ids[num_rows]; start = the rows' medoid.  Writes
 * out_dir/nav_index, nav_index.data and map.txt. */
int qv_build_nav(const void* rows, const int32_t* ids, int64_t num_rows, int32_t dim,
                 int32_t data_type, const qv_build_params* params, const char* out_dir);

/* GPU construction of the same index from a device array d_base [n][dim]
 * (Vamana with batched insertion; PQ trained on the device).  Returns a handle
 * whose graph, vectors and codes are already resident in HBM; qv_index_save
 * writes the three files. */
int qv_build_index_gpu(const void* d_base, int32_t data_type, int64_t n, int32_t dim,
                       const qv_build_params* params, int device, qv_index** out);

/* Writes <out_prefix>_disk.index, _pq_pivots.bin and _pq_compressed.bin of a
 * handle (device data copied back to the host). */
int qv_index_save(const qv_index* index, const char* out_prefix);

/* Copies a handle's data to caller host buffers (any may be NULL): the page
 * image [num_pages * 4096], codes [n][M], centroid [dim], pivots [256][dim],
 * chunk offsets [M+1] -- the heap-backend view host-side tools read. */
int qv_index_copy_out(const qv_index* index, uint8_t* pages, uint8_t* codes, float* centroid,
                      float* pivots, int32_t* chunk_offsets);

/* Brute-force exact top-k of each query over a device base array (fp32
 * arithmetic, exact for 8-bit data; ties broken by the smaller id).  All
 * pointers are device pointers; ids [nq][k] int32, dists [nq][k] f32. */
int qv_ground_truth(const void* d_base, int32_t data_type, int64_t n, int32_t dim,
                    const float* d_queries, int64_t nq, int32_t k, int32_t* d_ids,
                    float* d_dists, int device);

/* ---- Synthetic data: the seeded Gaussian mixture of the benchmark configs ----
 * Host generator (CPU) and device generator (HIP) produce identical values for
 * the same arguments.  uint8: centres uniform in [lo, hi], per-dim sigma, rounded
 * and clipped to [0, 255].  float: centres and noise standard normal, rows L2
 * normalised when normalize != 0.  Normal deviates are Irwin-Hall(12) sums of
 * counter-based 16-bit uniforms (exact in fp32), so the host and the device
 * produce the same uint8 rows bit for bit. */
typedef struct {
  uint64_t seed;
  int32_t num_centers;
  int32_t dim;
  int32_t data_type;     /* QV_UINT8 or QV_FLOAT */
  float center_lo, center_hi, sigma;
  int32_t normalize;
} qv_mixture;

int qv_mixture_fill_host(const qv_mixture* mix, int64_t first_row, int64_t rows,
                         void* dst);
int qv_mixture_fill_device(const qv_mixture* mix, int64_t first_row, int64_t rows,
                           void* d_dst, int device);

#ifdef __cplusplus
}
#endif
#endif
