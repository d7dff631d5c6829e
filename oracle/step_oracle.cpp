// TEST INFRASTRUCTURE: CPU restatement of the work around the loss head in one
// training step (rollout packing, gradient statistics, the Nesterov update). Only
// tests/ and bench.py's CPU-baseline leg load it, as the checker.
//
// Built with -ffp-contract=off: the reference (Zig, strict float mode) rounds every
// product and sum separately.
#include <cmath>
#include <cstdint>

extern "C" {

// src/optimizers/nesterov.zig:86-97 (mode 0) and nesterov_mlir.zig:93-99 (mode 1),
// element by element in f32, in place on p and v.
void oracle_nesterov(float* p, float* v, const float* g, int64_t n, float lr, float mu, int mode) {
  for (int64_t i = 0; i < n; ++i) {
    const float grad = g[i];
    const float p_master = p[i];
    if (mode == 0) {
      const float v_prev = v[i];
      const float v_new = mu * v_prev + grad;
      v[i] = v_new;
      p[i] = p_master - lr * (grad + mu * v_new);
    } else {
      const float v_new = mu * v[i] + lr * grad;
      v[i] = v_new;
      p[i] = p_master - v_new;
    }
  }
}

// src/nodes/controllers/rl_shepherd.zig:607-641, sequential like the reference.
void oracle_grad_stats(const float* g, int64_t n, double* sumsq, float* max_abs, int64_t* nan_count,
                       int64_t* inf_count) {
  double total = 0.0;
  float mx = 0.f;
  int64_t nans = 0, infs = 0;
  for (int64_t i = 0; i < n; ++i) {
    const float x = g[i];
    if (std::isnan(x)) {
      ++nans;
    } else if (std::isinf(x)) {
      ++infs;
    } else {
      total += static_cast<double>(x) * static_cast<double>(x);
      if (std::fabs(x) > mx) mx = std::fabs(x);
    }
  }
  *sumsq = total;
  *max_abs = mx;
  *nan_count = nans;
  *inf_count = infs;
}

// src/nodes/controllers/rl_shepherd.zig:487-515: row k gets rollout k's prompt then
// completion, up to seq_len tokens, mask 1 there; rows without a rollout stay zero.
// Returns -1 for offsets that decrease or run past a token array (those rows stay
// zero), else 0.
int oracle_pack(const int64_t* pt, int64_t npt, const int64_t* po, const int64_t* ct, int64_t nct,
                const int64_t* co, int64_t R, int64_t n_rows, int64_t T, int64_t* ids, float* mask) {
  int rc = 0;
  for (int64_t i = 0; i < n_rows * T; ++i) {
    ids[i] = 0;
    mask[i] = 0.f;
  }
  for (int64_t k = 0; k < R; ++k) {
    const int64_t p0 = po[k], p1 = po[k + 1], c0 = co[k], c1 = co[k + 1];
    if (p0 < 0 || p1 < p0 || p1 > npt || c0 < 0 || c1 < c0 || c1 > nct) {
      rc = -1;
      continue;
    }
    int64_t pos = 0;
    for (int64_t j = p0; j < p1 && pos < T; ++j, ++pos) {
      ids[k * T + pos] = pt[j];
      mask[k * T + pos] = 1.f;
    }
    for (int64_t j = c0; j < c1 && pos < T; ++j, ++pos) {
      ids[k * T + pos] = ct[j];
      mask[k * T + pos] = 1.f;
    }
  }
  return rc;
}

}  // extern "C"

extern "C" {

// src/core/math.zig:21-73, Sampler.sample with the uniform draw given: greedy
// (strict '>' argmax from index 0) for temperature < 1e-6, else the sequential f32
// max, sum of expf((l - max) / T), threshold u * sum and first crossing; falls back
// to n - 1 (:56).
int64_t oracle_sample(const float* logits, int64_t n, float temperature, float u) {
  if (temperature < 1e-6f) {
    float max_val = -INFINITY;
    int64_t max_idx = 0;
    for (int64_t i = 0; i < n; ++i)
      if (logits[i] > max_val) {
        max_val = logits[i];
        max_idx = i;
      }
    return max_idx;
  }
  float max_logit = -INFINITY;
  for (int64_t i = 0; i < n; ++i)
    if (logits[i] > max_logit) max_logit = logits[i];
  float sum_exp = 0.f;
  for (int64_t i = 0; i < n; ++i) sum_exp += std::exp((logits[i] - max_logit) / temperature);
  const float threshold = u * sum_exp;
  float cumulative = 0.f;
  for (int64_t i = 0; i < n; ++i) {
    cumulative += std::exp((logits[i] - max_logit) / temperature);
    if (cumulative >= threshold) return i;
  }
  return n - 1;
}

}  // extern "C"
