// qv_capi.cpp -- host-only C ABI entry points: error text, index construction,
// host-side synthetic data.
#include <cmath>
#include <cstring>
#include <exception>
#include <new>
#include <string>

#include <omp.h>

#include "qv_common.hpp"
#include "qv_mixture.hpp"

namespace qv {

namespace {
thread_local std::string g_last_error;

template <class F>
int host_guard(F&& f) {
  try {
    f();
    return QV_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.code;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return QV_ENOMEM;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return QV_EIO;
  }
}
}  // namespace

void set_last_error(const std::string& msg) { g_last_error = msg; }

void build_index_cpu(const void* base, int dtype, int64_t n, int dim, const qv_build_params& prm,
                     const std::string& prefix);
void build_nav_cpu(const void* rows, const int32_t* ids, int64_t s, int dim, int dtype, const qv_build_params& prm,
                   const std::string& dir);

}  // namespace qv

extern "C" {

const char* qv_last_error(void) { return qv::g_last_error.c_str(); }

void qv_build_params_default(qv_build_params* p) {
  if (!p) return;
  std::memset(p, 0, sizeof(*p));
  p->R = 64;
  p->L = 100;
  p->alpha = 1.2f;
  p->num_chunks = 32;
  p->kmeans_iters = 15;
  p->pq_train_max = 262144;
  p->seed = 0x5EED5EEDull;
  p->threads = 0;
  p->passes = 2;
}

int qv_build_index_cpu(const void* base, int32_t data_type, int64_t n, int32_t dim,
                       const qv_build_params* params, const char* out_prefix) {
  return qv::host_guard([&] {
    if (!base || !out_prefix || dim <= 0) qv::fail(QV_EINVAL, "bad argument");
    if (data_type != QV_UINT8 && data_type != QV_FLOAT && data_type != QV_INT8)
      qv::fail(QV_EINVAL, "bad data type");
    qv_build_params p;
    qv_build_params_default(&p);
    if (params) p = *params;
    qv::build_index_cpu(base, data_type, n, dim, p, out_prefix);
  });
}

int qv_build_nav(const void* rows, const int32_t* ids, int64_t num_rows, int32_t dim, int32_t data_type,
                 const qv_build_params* params, const char* out_dir) {
  return qv::host_guard([&] {
    if (!rows || !ids || !out_dir || dim <= 0) qv::fail(QV_EINVAL, "bad argument");
    if (data_type != QV_UINT8 && data_type != QV_FLOAT && data_type != QV_INT8)
      qv::fail(QV_EINVAL, "bad data type");
    qv_build_params p;
    qv_build_params_default(&p);
    p.R = 28;
    p.L = 64;
    if (params) p = *params;
    qv::build_nav_cpu(rows, ids, num_rows, dim, data_type, p, out_dir);
  });
}

int qv_find_index_files(const char* index_dir, char* index_file, char* pq_prefix, int32_t capacity) {
  return qv::host_guard([&] {
    if (!index_dir || !index_file || !pq_prefix || capacity <= 0) qv::fail(QV_EINVAL, "bad argument");
    const std::string a = qv::find_index_file(index_dir);
    const std::string b = qv::find_pq_prefix(index_dir);
    if ((int64_t)a.size() >= capacity || (int64_t)b.size() >= capacity) qv::fail(QV_EINVAL, "path buffer too small");
    std::memcpy(index_file, a.c_str(), a.size() + 1);
    std::memcpy(pq_prefix, b.c_str(), b.size() + 1);
  });
}

int qv_read_layout(const char* index_file, const char* data_type, qv_index_info* out) {
  return qv::host_guard([&] {
    if (!index_file || !data_type || !out) qv::fail(QV_EINVAL, "null argument");
    const qv::Layout L = qv::parse_diskann_metadata(index_file, qv::parse_data_type(data_type));
    std::memset(out, 0, sizeof(*out));
    out->num_data = L.num_data;
    out->num_dims = L.num_dims;
    out->max_m0 = L.max_m0;
    out->enter_point = L.enter_point;
    out->data_size = L.data_size;
    out->node_size = L.node_size;
    out->num_pages = L.num_pages;
    out->nodes_per_page = L.nodes_per_page;
    out->data_type = L.data_type;
  });
}

int qv_read_index_pages(const char* index_file, int64_t num_pages, uint8_t* dst) {
  return qv::host_guard([&] {
    if (!index_file || !dst || num_pages < 0) qv::fail(QV_EINVAL, "bad argument");
    qv::read_index_pages(index_file, num_pages, dst);
  });
}

int qv_mixture_fill_host(const qv_mixture* m, int64_t first_row, int64_t rows, void* dst) {
  return qv::host_guard([&] {
    if (!m || !dst || rows < 0 || m->dim <= 0 || m->num_centers <= 0) qv::fail(QV_EINVAL, "bad argument");
    if (m->data_type == QV_UINT8) {
      uint8_t* out = static_cast<uint8_t*>(dst);
#pragma omp parallel for schedule(static)
      for (int64_t r = 0; r < rows; r++)
        for (int32_t j = 0; j < m->dim; j++)
          out[r * m->dim + j] = qv::mixture_u8(m->seed, m->num_centers, m->dim, m->center_lo,
                                               m->center_hi, m->sigma, first_row + r, j);
    } else if (m->data_type == QV_FLOAT) {
      float* out = static_cast<float*>(dst);
#pragma omp parallel for schedule(static)
      for (int64_t r = 0; r < rows; r++) {
        float* row = out + r * m->dim;
        double ss = 0.0;
        for (int32_t j = 0; j < m->dim; j++) {
          const float v = qv::mixture_f32_raw(m->seed, m->num_centers, m->dim, m->sigma, first_row + r, j);
          row[j] = v;
          const double dv = (double)v;
          ss = ss + dv * dv;
        }
        if (m->normalize) {
          const double inv = 1.0 / std::sqrt(ss);
          for (int32_t j = 0; j < m->dim; j++) row[j] = (float)((double)row[j] * inv);
        }
      }
    } else {
      qv::fail(QV_EINVAL, "mixture data_type must be uint8 or float");
    }
  });
}

}  // extern "C"
