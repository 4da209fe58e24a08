// quiver_search -- command-line front end with the reference's flags, stdout
// report and result files (bin/quiver_search.cu:58-320, bin/common/*.hpp),
// running the memory (heap) backend through libquiver_hip's C ABI.
#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <map>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "quiver_hip.h"

namespace {

struct Flag {
  std::string value;
  bool used = false;
  bool is_bool = false;
};

const char* kUsage =
    "Usage: quiver_search --index-dir DIR --query FILE --data-type {uint8,int8,float}\n"
    "  [--topk 10] [--ef-search 30] [--repeat 20] [--ground-truth FILE]\n"
    "  [--memory-backend heap|mmap] [--memory-index-file FILE] [--ssd-list-file FILE]\n"
    "  [--graph-placement hbm|host] [--search-kernel auto|lut|shared-pivots]\n"
    "  [--num-blocks N (default: fill the GPU)] [--num-blocks-list L] [--pipe-width 2] [--queries-per-block 1]\n"
    "  [--poll-threads 6] [--runners-per-ssd 1] [--early-exit-policy gpruning|none]\n"
    "  [--result-prefix P] [--final-recall-csv F] [--skip-nav] [--help]\n"
    "  [--per-step-recall [--recall-threshold 0.9] [--step-recall-csv quiver_step_recall.csv]]\n"
    "  [--static-batches] [--neighbour-codes]\n";

bool parse_int(const std::string& s, int& out) {
  char* end = nullptr;
  errno = 0;
  long v = std::strtol(s.c_str(), &end, 10);
  if (errno || end == s.c_str() || *end) return false;
  out = (int)v;
  return true;
}

template <class T>
std::vector<T> read_bin(const std::string& path, int32_t& n, int32_t& d) {
  std::ifstream in(path, std::ios::binary);
  if (!in.is_open()) {
    std::cerr << "Failed to open file " << path << std::endl;
    std::exit(1);
  }
  in.read(reinterpret_cast<char*>(&n), 4);
  in.read(reinterpret_cast<char*>(&d), 4);
  std::vector<T> v((size_t)n * (size_t)d);
  in.read(reinterpret_cast<char*>(v.data()), (std::streamsize)(sizeof(T) * v.size()));
  if (!in) {
    std::cerr << "Truncated file " << path << std::endl;
    std::exit(1);
  }
  return v;
}

// load_queries_as_float (bin/common/data_io.hpp:73-108): the element type
// follows the file suffix; the whole set is repeated `repeat` times.
std::vector<float> load_queries(const std::string& path, int repeat, int32_t& n, int32_t& d) {
  std::vector<float> q;
  if (path.find(".u8bin") != std::string::npos) {
    auto raw = read_bin<uint8_t>(path, n, d);
    q.assign(raw.begin(), raw.end());
  } else if (path.find(".i8bin") != std::string::npos) {
    auto raw = read_bin<int8_t>(path, n, d);
    q.assign(raw.begin(), raw.end());
  } else {
    q = read_bin<float>(path, n, d);
  }
  if (repeat > 1) {
    std::vector<float> r;
    r.reserve(q.size() * (size_t)repeat);
    for (int i = 0; i < repeat; i++) r.insert(r.end(), q.begin(), q.end());
    q.swap(r);
    n *= repeat;
  }
  return q;
}

template <class T>
void write_result(const std::string& path, const T* v, int32_t n, int32_t k) {
  std::ofstream out(path, std::ios::binary | std::ios::trunc);
  if (!out.is_open()) throw std::runtime_error("Failed to open binary result file " + path);
  out.write(reinterpret_cast<const char*>(&n), 4);
  out.write(reinterpret_cast<const char*>(&k), 4);
  out.write(reinterpret_cast<const char*>(v), (std::streamsize)(sizeof(T) * (size_t)n * (size_t)k));
  if (!out) throw std::runtime_error("Failed to write binary result file " + path);
}

// calc_recall / calc_one_query_recall (bin/common/recall.hpp:15-62).
int query_hits(const int32_t* res, const int32_t* gt, int k) {
  std::set<int32_t> e(gt, gt + k);
  int h = 0;
  for (int j = 0; j < k; j++) h += e.count(res[j]) ? 1 : 0;
  return h;
}

}  // namespace

// write_step_recall_csv (src/quiver/search.cu:100-153): one row per query and
// the reached / step-percentile summary lines.
bool write_step_recall(const std::string& path, const std::vector<int32_t>& steps,
                       const std::vector<int32_t>& hits, int topk, float threshold) {
  std::ofstream out(path);
  if (!out.is_open()) {
    std::cerr << "Failed to open step recall CSV " << path << std::endl;
    return false;
  }
  out << "query_id,step,hits,recall,reached\n";
  std::vector<int32_t> reached;
  for (size_t q = 0; q < steps.size(); q++) {
    const bool ok = steps[q] >= 0;
    if (ok) reached.push_back(steps[q]);
    out << q << "," << steps[q] << "," << hits[q] << "," << std::fixed << std::setprecision(6)
        << (double)hits[q] / (double)topk << "," << (ok ? 1 : 0) << "\n";
  }
  out.close();
  std::sort(reached.begin(), reached.end());
  const int required = std::max(1, std::min(topk, (int)std::ceil(threshold * (float)topk - 1e-6f)));
  std::cout << "[Quiver] Step recall CSV: " << path << "\n"
            << "[Quiver] Step recall reached=" << reached.size() << " unreached=" << steps.size() - reached.size()
            << " threshold=" << threshold << " required_hits=" << required << std::endl;
  if (!reached.empty()) {
    auto pct = [&](double p) {
      size_t i = (size_t)((double)reached.size() * p / 100.0);
      if (i >= reached.size()) i = reached.size() - 1;
      return (double)reached[i];
    };
    std::cout << "[Quiver] Step recall steps p50=" << pct(50) << " p90=" << pct(90) << " p99=" << pct(99)
              << " max=" << reached.back() << std::endl;
  }
  return true;
}

int main(int argc, char** argv) {
  std::map<std::string, Flag> f;
  const char* value_flags[] = {"--index-dir", "--query", "--topk", "--ground-truth", "--data-type",
                               "--ef-search", "--ssd-list-file", "--memory-backend",
                               "--memory-index-file", "--repeat", "--num-blocks", "--poll-threads",
                               "--spdk-submit-queue-cap", "--spdk-task-contexts",
                               "--spdk-runner-io-contexts", "--pipe-width", "--queries-per-block",
                               "--runners-per-ssd", "--num-blocks-list", "--recall-threshold",
                               "--step-recall-csv", "--final-recall-csv", "--result-prefix",
                               "--early-exit-policy", "--graph-placement", "--search-kernel"};
  const char* bool_flags[] = {"--skip-nav", "--per-step-recall", "--static-batches", "--neighbour-codes",
                              "--help"};
  for (auto* s : value_flags) f[s] = Flag{};
  for (auto* s : bool_flags) f[s] = Flag{"", false, true};
  f["--topk"].value = "10";
  f["--ef-search"].value = "30";
  f["--repeat"].value = "20";
  f["--memory-backend"].value = "heap";
  // Unset, --num-blocks fills the GPU with query slots (0 below); a value
  // given is the slot count, validated as the reference validates it.  The
  // count changes only how many queries run at once, never their results.
  f["--num-blocks"].value = "0";
  f["--poll-threads"].value = "6";
  f["--pipe-width"].value = "2";
  f["--queries-per-block"].value = "1";
  f["--runners-per-ssd"].value = "1";
  f["--early-exit-policy"].value = "gpruning";
  f["--graph-placement"].value = "hbm";
  f["--search-kernel"].value = "auto";
  for (int i = 1; i < argc; i++) {
    std::string a = argv[i];
    auto it = f.find(a);
    if (it == f.end()) {
      std::cerr << "Unknown argument: " << a << "\n" << kUsage;
      return 1;
    }
    it->second.used = true;
    if (it->second.is_bool) continue;
    if (i + 1 >= argc) {
      std::cerr << a << ": expected 1 argument(s). 0 provided.\n" << kUsage;
      return 1;
    }
    it->second.value = argv[++i];
  }
  if (f["--help"].used) {
    std::cout << kUsage;
    return 0;
  }
  for (const char* req : {"--index-dir", "--query", "--data-type"}) {
    if (!f[req].used) {
      std::cerr << req << ": required.\n" << kUsage;
      return 1;
    }
  }
  int topk = 0, ef = 0, repeat = 0, num_blocks = 0, poll = 0, pipe_w = 0, qpb = 0, rps = 0;
  struct {
    const char* name;
    int* dst;
  } ints[] = {{"--topk", &topk}, {"--ef-search", &ef}, {"--repeat", &repeat},
              {"--num-blocks", &num_blocks}, {"--poll-threads", &poll}, {"--pipe-width", &pipe_w},
              {"--queries-per-block", &qpb}, {"--runners-per-ssd", &rps}};
  for (auto& e : ints) {
    if (!parse_int(f[e.name].value, *e.dst)) {
      std::cerr << "invalid integer for " << e.name << ": " << f[e.name].value << "\n" << kUsage;
      return 1;
    }
  }
  // bin/common/cli_shared.hpp: SPDK needs a build with SPDK; this one has none.
  if (f["--ssd-list-file"].used) {
    std::ifstream sl(f["--ssd-list-file"].value);
    std::string line;
    bool any = false;
    while (sl >> line) any = true;
    if (any) {
      std::cerr << "This binary was built without SPDK support" << std::endl;
      return 1;
    }
  }
  // bin/common/cli_validation.hpp:9-30
  if (f["--num-blocks"].used && num_blocks <= 0) {
    std::cerr << "--num-blocks must be positive" << std::endl;
    return 1;
  }
  if (poll <= 0) { std::cerr << "--poll-threads must be positive" << std::endl; return 1; }
  if (pipe_w < 1 || pipe_w > 16) { std::cerr << "--pipe-width must be in [1, 16]" << std::endl; return 1; }
  if (qpb < 1 || qpb > 8) { std::cerr << "--queries-per-block must be in [1, 8]" << std::endl; return 1; }
  const std::string policy = f["--early-exit-policy"].value;
  if (policy != "none" && policy != "gpruning") {
    std::cerr << "invalid --early-exit-policy: " << policy << " (expected gpruning or none)" << std::endl;
    return 1;
  }
  // --per-step-recall (bin/quiver_search.cu:219-233): the ground truth stops
  // each query once its top-k reaches the threshold
  const bool step_recall = f["--per-step-recall"].used;
  float recall_threshold = 0.9f;
  const std::string step_csv = f["--step-recall-csv"].used ? f["--step-recall-csv"].value : "quiver_step_recall.csv";
  std::vector<int32_t> step_gt;
  int32_t step_gt_n = 0, step_gt_w = 0;
  if (f["--recall-threshold"].used) {
    char* end = nullptr;
    recall_threshold = std::strtof(f["--recall-threshold"].value.c_str(), &end);
    if (end == f["--recall-threshold"].value.c_str() || *end != 0) {
      std::cerr << "invalid float for --recall-threshold: " << f["--recall-threshold"].value << "\n" << kUsage;
      return 1;
    }
  }
  if (step_recall) {
    if (!f["--ground-truth"].used) {
      std::cerr << "--per-step-recall requires --ground-truth" << std::endl;
      return 1;
    }
    if (pipe_w != 1 || qpb != 1) {
      std::cerr << "--per-step-recall currently requires pipe_width=1 and queries_per_block=1" << std::endl;
      return 1;
    }
    try {
      step_gt = read_bin<int32_t>(f["--ground-truth"].value, step_gt_n, step_gt_w);
    } catch (const std::exception& e) {
      std::cerr << e.what() << std::endl;
      return 1;
    }
    std::cout << "[Quiver] per-step recall enabled: threshold=" << recall_threshold << " csv=" << step_csv
              << " gt_count=" << step_gt_n << " gt_width=" << step_gt_w << std::endl;
  }
  std::vector<int> nb_list{num_blocks};
  if (f["--num-blocks-list"].used) {
    nb_list.clear();
    std::string raw = f["--num-blocks-list"].value;
    for (char& c : raw) if (c == ',') c = ' ';
    std::istringstream is(raw);
    std::string tok;
    while (is >> tok) {
      int v = 0;
      if (!parse_int(tok, v)) {
        std::cerr << "invalid integer in --num-blocks-list: " << tok << std::endl;
        return 1;
      }
      if (v <= 0) {
        std::cerr << "--num-blocks-list values must be positive: " << v << std::endl;
        return 1;
      }
      nb_list.push_back(v);
    }
    if (nb_list.empty()) {
      std::cerr << "empty list for --num-blocks-list" << std::endl;
      return 1;
    }
  }
  const std::string prefix = f["--result-prefix"].value;
  if (!prefix.empty() && nb_list.size() != 1) {
    std::cerr << "--result-prefix cannot be combined with a multi-value --num-blocks-list" << std::endl;
    return 1;
  }
  std::cout << "[Quiver] runners_per_ssd=" << rps << (f["--runners-per-ssd"].used ? " (cli)" : "") << std::endl;
  std::cout << "[Quiver] early-exit policy=" << policy << std::endl;

  const std::string kname = f["--search-kernel"].value;
  const int32_t kernel = kname == "lut" ? QV_KERNEL_LUT
                         : kname == "shared-pivots" ? QV_KERNEL_SHARED_PIVOTS
                         : kname == "auto" ? QV_KERNEL_AUTO : -1;
  if (kernel < 0) {
    std::cerr << "--search-kernel must be auto, lut or shared-pivots" << std::endl;
    return 1;
  }
  qv_index* ix = nullptr;
  const char* mem_file = f["--memory-index-file"].used ? f["--memory-index-file"].value.c_str() : nullptr;
  const std::string placement = f["--graph-placement"].value;
  if (placement != "hbm" && placement != "host") {
    std::cerr << "--graph-placement must be hbm or host" << std::endl;
    return 1;
  }
  if (qv_index_open_ex(f["--index-dir"].value.c_str(), f["--data-type"].value.c_str(),
                       f["--memory-backend"].value.c_str(), mem_file, 0,
                       placement == "host" ? QV_GRAPH_HOST : QV_GRAPH_HBM, &ix) != QV_OK) {
    std::cerr << qv_last_error() << std::endl;
    return 1;
  }
  // each node's neighbours' code rows as one block in HBM: the same results,
  // fewer bytes per hop, n * R * M bytes of device memory
  if (f["--neighbour-codes"].used && qv_index_neighbour_codes(ix, 1) != QV_OK) {
    std::cerr << qv_last_error() << std::endl;
    qv_index_close(ix);
    return 1;
  }
  qv_index_info info;
  qv_index_get_info(ix, &info);
  int32_t nq = 0, dim = 0;
  std::vector<float> queries = load_queries(f["--query"].value, repeat, nq, dim);
  if (dim != info.num_dims) {
    std::cerr << "Query dimension mismatch: query file '" << f["--query"].value << "' has " << dim
              << " dims, but the index expects " << info.num_dims << " dims" << std::endl;
    qv_index_close(ix);
    return 1;
  }
  if (f["--skip-nav"].used)
    std::cout << "[Quiver] --skip-nav enabled: nav graph disabled; all queries start from global enter_point="
              << info.enter_point << std::endl;

  std::vector<int32_t> ids((size_t)nq * topk), found((size_t)nq), hops((size_t)nq);
  std::vector<float> dists((size_t)nq * topk);
  for (int nb : nb_list) {
    qv_search_opts o;
    qv_search_opts_default(&o);
    o.num_blocks = nb;
    o.queries_per_block = qpb;
    o.pipe_width = pipe_w;
    o.early_exit = policy == "gpruning" ? QV_EXIT_GPRUNING : QV_EXIT_NONE;
    o.gpruning_warmup = 10;
    o.gpruning_patience = 8;
    o.skip_nav = f["--skip-nav"].used ? 1 : 0;
    o.kernel = kernel;
    const bool static_batches = f["--static-batches"].used;
    if (static_batches) {  // run_static_batch_search (search.cu:1703-1796)
      o.admission = QV_ADMIT_STATIC;
      // With --num-blocks unset (0) the library fills the GPU with slots; the
      // batch line then follows the search, from the slots it launched.
      if (nb > 0) {
        const int64_t stride = (int64_t)nb * qpb;
        std::cout << "[Quiver] StaticBatch: " << (nq + stride - 1) / stride << " batches of " << nb
                  << " blocks x Q=" << qpb << " = " << stride << " queries per batch, total " << nq << " queries"
                  << std::endl;
      }
    }
    if (const char* e = std::getenv("QUIVER_PREFEED")) o.prefeed = std::atoi(e);
    if (const char* e = std::getenv("QUIVER_ADMIT_MIN_BATCH")) o.admit_min_batch = std::max(1, std::atoi(e));
    std::vector<int32_t> sr_step, sr_hits;
    if (step_recall) {
      sr_step.resize((size_t)nq);
      sr_hits.resize((size_t)nq);
      o.step_recall_gt = step_gt.data();
      o.step_recall_gt_width = step_gt_w;
      o.step_recall_gt_count = step_gt_n;
      o.step_recall_threshold = recall_threshold;
      o.step_recall_step = sr_step.data();
      o.step_recall_hits = sr_hits.data();
    }
    qv_search_report rep;
    if (qv_search(ix, queries.data(), nq, dim, topk, ef, &o, ids.data(), dists.data(), found.data(), &rep) != QV_OK) {
      std::cerr << qv_last_error() << std::endl;
      qv_index_close(ix);
      return 1;
    }
    qv_last_hops(ix, hops.data(), nq);
    if (static_batches && nb <= 0) {
      // max_inflight of a static search is its batch size: min(nq, slots)
      const int64_t stride = std::max<int64_t>(1, rep.max_inflight);
      std::cout << "[Quiver] StaticBatch: " << (nq + stride - 1) / stride << " batches of " << stride
                << " queries (query slots filling the GPU, Q=" << qpb << "), total " << nq << " queries"
                << std::endl;
    }
    if (step_recall && !write_step_recall(step_csv, sr_step, sr_hits, topk, recall_threshold)) {
      qv_index_close(ix);
      return 1;
    }
    std::cout << "[Quiver] search_kernel="
              << (rep.kernel == QV_KERNEL_SHARED_PIVOTS ? "shared-pivots" : "lut") << std::endl;
    // format_run_report (src/shared/common/run_report.hpp:96-140)
    std::ostringstream os;
    os << std::fixed;
    os << "========== Quiver Result ==========\n";
    os << "Query Params:\n  topk=" << topk << " ef_search=" << ef << " repeat=" << repeat
       << " data_type=" << f["--data-type"].value << "\n";
    os << "Runtime Params:\n  num_blocks=" << rep.num_blocks << " pipe_width=" << pipe_w
       << " queries_per_block=" << qpb << " task_slots=" << rep.num_blocks
       << " max_inflight=" << rep.max_inflight << " backend=hbm\n\n";
    os << "Performance:\n  QPS: " << std::setprecision(2) << rep.qps << "\n";
    os << "  QueryLatency(ms): avg=" << std::setprecision(3) << rep.lat_avg_ms << " p50=" << rep.lat_p50_ms
       << " p90=" << rep.lat_p90_ms << " p99=" << rep.lat_p99_ms << " p99.9=" << rep.lat_p999_ms
       << " max=" << rep.lat_max_ms << "\n";
    os << "  SSD Avg Bandwidth: 0.00 GB/s\n  SSD Avg IOPS: 0\n";
    os << "===================================\n";
    std::printf("%s", os.str().c_str());
    double hop_sum = 0;
    for (int32_t h : hops) hop_sum += h;
    std::cout << "[Quiver] Finish summary: policy=" << policy << " avg_finish_step=" << std::fixed
              << std::setprecision(2) << hop_sum / nq << " finished=" << nq << "/" << nq;
    if (policy == "gpruning")
      std::cout << " stopped=" << rep.early_stopped << "/" << nq << " ("
                << 100.0 * rep.early_stopped / nq << "%)";
    std::cout << std::defaultfloat << std::endl;

    if (f["--ground-truth"].used) {
      int32_t gn = 0, gw = 0;
      auto gt = read_bin<int32_t>(f["--ground-truth"].value, gn, gw);
      if (gw < topk) {
        std::cerr << "ground truth width " << gw << " < topk " << topk << std::endl;
        qv_index_close(ix);
        return 1;
      }
      int64_t hits = 0;
      for (int32_t i = 0; i < gn && i < nq; i++) hits += query_hits(&ids[(size_t)i * topk], &gt[(size_t)i * gw], topk);
      std::printf("Recall @ %d: %lf\n", topk, (double)hits / ((double)gn * topk));
      const std::string csv = f["--final-recall-csv"].value;
      if (!csv.empty()) {
        std::ofstream out(csv);
        out << "query_id,gt_query_id,hits,recall\n";
        for (int32_t i = 0; i < nq; i++) {
          const int32_t g = i % gn;
          const int h = query_hits(&ids[(size_t)i * topk], &gt[(size_t)g * gw], topk);
          out << i << "," << g << "," << h << "," << std::fixed << std::setprecision(6)
              << (double)h / topk << "\n";
        }
        std::cout << "[Quiver] Per-query recall CSV: " << csv << std::endl;
      }
    }
    if (!prefix.empty()) {
      try {
        write_result(prefix + "_ids.bin", ids.data(), nq, topk);
        write_result(prefix + "_distances.bin", dists.data(), nq, topk);
      } catch (const std::exception& e) {
        std::cerr << e.what() << std::endl;
        qv_index_close(ix);
        return 1;
      }
      std::cout << "[Quiver] Search results: " << prefix << "_ids.bin " << prefix << "_distances.bin" << std::endl;
    }
  }
  qv_index_close(ix);
  return 0;
}
