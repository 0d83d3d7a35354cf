// gmoe_predict.cpp — expert-activation predictor (host code).
//
// garuda/src/predictor/mod.rs:15-134: a first-order Markov model over global expert ids
// (layer * n_experts + expert). observe(prev, next) adds one to C[p][q] for every pair
// (saturating); predict(current, k) scores each q by the sum over p in current of
// C[p][q], drops zero scores, orders by score (descending) then id (ascending) and keeps
// k; score(predicted, actual) counts correct / wasted / missed. The transition table is
// n_experts^2 u32 counts, behind a reader-writer lock.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <shared_mutex>
#include <vector>

#include "../../include/garuda_moe.h"

namespace gmoe {
void set_last_error(const char* msg);  // gmoe_api.cpp
}

struct gmoe_predictor {
  uint32_t n = 1;
  std::vector<uint32_t> counts;  // [n][n]
  mutable std::shared_mutex mu;
  gmoe_predict_stats stats{};
  std::mutex stats_mu;
};

namespace {

gmoe_status pfail(gmoe_status s, const char* msg) {
  gmoe::set_last_error(msg);
  return s;
}

}  // namespace

namespace gmoe {

// predict without taking the lock (the caller holds it)
void predict_locked(const gmoe_predictor* p, const uint32_t* cur, uint32_t nc, uint32_t k, std::vector<uint32_t>* out) {
  out->clear();
  if (nc == 0 || k == 0) return;
  const uint32_t n = p->n;
  std::vector<uint64_t> score(n, 0);
  for (uint32_t i = 0; i < nc; i++) {
    const uint32_t q0 = cur[i];
    if (q0 >= n) continue;
    const uint32_t* row = p->counts.data() + (size_t)q0 * n;
    for (uint32_t q = 0; q < n; q++) score[q] += row[q];
  }
  std::vector<uint32_t> ids;
  for (uint32_t q = 0; q < n; q++)
    if (score[q] > 0) ids.push_back(q);
  std::sort(ids.begin(), ids.end(), [&](uint32_t a, uint32_t b) { return score[a] != score[b] ? score[a] > score[b] : a < b; });
  if (ids.size() > k) ids.resize(k);
  *out = std::move(ids);
}

void observe_locked(gmoe_predictor* p, const uint32_t* prev, uint32_t np, const uint32_t* next, uint32_t nn) {
  const uint32_t n = p->n;
  for (uint32_t i = 0; i < np; i++)
    for (uint32_t j = 0; j < nn; j++) {
      const uint32_t a = prev[i], b = next[j];
      if (a < n && b < n) {
        uint32_t& c = p->counts[(size_t)a * n + b];
        if (c != UINT32_MAX) c++;
      }
    }
}

void score_counts(gmoe_predictor* p, const uint32_t* pred, uint32_t np, const uint32_t* act, uint32_t na) {
  std::lock_guard<std::mutex> g(p->stats_mu);
  for (uint32_t i = 0; i < np; i++) {
    if (std::find(act, act + na, pred[i]) != act + na) p->stats.correct++;
    else p->stats.wasted++;
  }
  for (uint32_t i = 0; i < na; i++)
    if (std::find(pred, pred + np, act[i]) == pred + np) p->stats.missed++;
}

}  // namespace gmoe

extern "C" {

gmoe_status gmoe_predictor_create(uint32_t n_experts, gmoe_predictor** out) {
  if (!out) return pfail(GMOE_ERR_INFERENCE, "null output pointer");
  const uint32_t n = std::max(1u, n_experts);
  if ((uint64_t)n * n > (1ull << 32)) return pfail(GMOE_ERR_CONFIG, "predictor of more than 65536 experts");
  auto* p = new (std::nothrow) gmoe_predictor;
  if (!p) return pfail(GMOE_ERR_CONFIG, "out of host memory");
  p->n = n;
  try {
    p->counts.assign((size_t)n * n, 0);
  } catch (const std::bad_alloc&) {
    delete p;
    return pfail(GMOE_ERR_CONFIG, "out of host memory for the transition table");
  }
  *out = p;
  return GMOE_OK;
}

void gmoe_predictor_destroy(gmoe_predictor* p) { delete p; }

gmoe_status gmoe_predictor_observe(gmoe_predictor* p, const uint32_t* prev, uint32_t np, const uint32_t* next,
                                   uint32_t nn) {
  if (!p || (np && !prev) || (nn && !next)) return pfail(GMOE_ERR_INFERENCE, "null predictor or ids");
  std::unique_lock<std::shared_mutex> g(p->mu);
  gmoe::observe_locked(p, prev, np, next, nn);
  return GMOE_OK;
}

gmoe_status gmoe_predictor_predict(const gmoe_predictor* p, const uint32_t* cur, uint32_t nc, uint32_t k,
                                   uint32_t* out, uint32_t* n_out) {
  if (!p || !n_out || (nc && !cur) || (k && !out)) return pfail(GMOE_ERR_INFERENCE, "null predictor, ids or output");
  std::vector<uint32_t> ids;
  {
    std::shared_lock<std::shared_mutex> g(p->mu);
    gmoe::predict_locked(p, cur, nc, k, &ids);
  }
  std::copy(ids.begin(), ids.end(), out);
  *n_out = (uint32_t)ids.size();
  return GMOE_OK;
}

gmoe_status gmoe_predictor_score(gmoe_predictor* p, const uint32_t* pred, uint32_t np, const uint32_t* act,
                                 uint32_t na) {
  if (!p || (np && !pred) || (na && !act)) return pfail(GMOE_ERR_INFERENCE, "null predictor or ids");
  gmoe::score_counts(p, pred, np, act, na);
  return GMOE_OK;
}

gmoe_status gmoe_predictor_stats(const gmoe_predictor* p, gmoe_predict_stats* out) {
  if (!p || !out) return pfail(GMOE_ERR_INFERENCE, "null predictor or output");
  std::lock_guard<std::mutex> g(const_cast<gmoe_predictor*>(p)->stats_mu);
  *out = p->stats;
  return GMOE_OK;
}

gmoe_status gmoe_predictor_get_counts(const gmoe_predictor* p, uint32_t* counts, uint64_t n) {
  if (!p || !counts) return pfail(GMOE_ERR_INFERENCE, "null predictor or buffer");
  if (n != (uint64_t)p->n * p->n) return pfail(GMOE_ERR_INFERENCE, "table size is n_experts^2");
  std::shared_lock<std::shared_mutex> g(p->mu);
  std::memcpy(counts, p->counts.data(), n * 4);
  return GMOE_OK;
}

gmoe_status gmoe_predictor_set_counts(gmoe_predictor* p, const uint32_t* counts, uint64_t n) {
  if (!p || !counts) return pfail(GMOE_ERR_INFERENCE, "null predictor or buffer");
  if (n != (uint64_t)p->n * p->n) return pfail(GMOE_ERR_INFERENCE, "table size is n_experts^2");
  std::unique_lock<std::shared_mutex> g(p->mu);
  std::memcpy(p->counts.data(), counts, n * 4);
  return GMOE_OK;
}

}  // extern "C"
