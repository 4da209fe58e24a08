// Exports the reference's recall routines (bin/common/recall.hpp:15-62, compiled
// from the reference checkout by `make ref`) with C linkage so tests can compare
// the oracle's restatement against the reference's own code.
#include "common/recall.hpp"

extern "C" double ref_calc_recall(const int* results, const int* gt, long nq,
                                  long gt_width, int topk) {
  return bin_common::calc_recall(results, gt, (size_t)nq, (size_t)gt_width, topk);
}

extern "C" int ref_query_hits(const int* results, const int* gt, int topk) {
  return bin_common::calc_one_query_recall(results, gt, topk).hits;
}
