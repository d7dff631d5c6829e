// TEST INFRASTRUCTURE — the CPU oracle of the GRPO loss head. Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
// as the checker (or the timed CPU baseline), never as the product path.
//
// It restates the reference's computation on the CPU:
//   * the loss graph of tools/export_qwen_forward.py:146-163, in the StableHLO op
//     order of its cross-entropy lowering, models/tests/qwen_test.mlir:257-286
//     (reduce max -> subtract -> exp -> reduce add -> log -> subtract -> gather
//     -> negate -> select on id != -100);
//   * the group advantages of src/nodes/controllers/rl_shepherd.zig:462-479,
//     bit-exactly (sequential fp32, no contraction, IEEE div/sqrt);
//   * the reference autodiff backward of that graph with its numeric guards
//     (precision = kFaithful): divideVJP adds 1e-4 to every divisor
//     (src/autodiff/vjp_rules.zig:197-203), logVJP divides by S + 1e-4
//     (vjp_rules.zig:1509-1521), expVJP multiplies by a recomputed exp
//     (vjp_rules.zig:1436-1473), reduceMaxVJP routes -sum(ds) to every element
//     equal to the row max (vjp_rules.zig:673-775), and every edge is
//     finite-guarded and clamped to [-100, 100] (src/autodiff/engine.zig:604-681,
//     bounds src/compiler/graph_builder.zig:335-337);
//   * the clipped-ratio + k3-KL loss, which has no reference counterpart, in
//     closed form.
// Precision kExact computes everything in double from the (exactly widened)
// inputs and is the truth the tolerances are measured against.
//
// Build: make -C oracle  ->  oracle/libpcp_oracle.so  (g++ -O3 -fopenmp
// -ffp-contract=off; the advantage restatement relies on no FMA contraction).

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include <omp.h>

namespace {

enum Dtype { kF16 = 0, kBF16 = 1, kF32 = 2, kF64 = 3 };
enum Precision { kExact = 0, kRefOrderF32 = 1, kFaithful = 2 };
enum LossMode { kReinforce = 0, kClipKl = 1 };

// bf16 -> f32 is exact: the 16 bits are the high half of the f32 pattern.
inline float bf16_to_f32(uint16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// f32 -> bf16, round to nearest, ties to even; NaN stays a quiet NaN.
inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return static_cast<uint16_t>(u >> 16);
}

// IEEE binary16 -> f32 (exact).
inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else {  // subnormal: renormalise
      int e = -1;
      do {
        ++e;
        man <<= 1;
      } while ((man & 0x400u) == 0);
      u = sign | (static_cast<uint32_t>(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Element i of a logits array as a double (exact for every supported dtype);
// kF64 inputs carry logits computed exactly elsewhere (e.g. hidden * W^T in f64).
inline double loadd(const void* p, int dt, int64_t i) {
  switch (dt) {
    case kBF16: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case kF16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    case kF64: return static_cast<const double*>(p)[i];
    default: return static_cast<const float*>(p)[i];
  }
}
// The same element rounded to f32 (the reference graph runs in f32).
inline float load(const void* p, int dt, int64_t i) { return static_cast<float>(loadd(p, dt, i)); }

// Guard + clamp of one gradient edge (engine.zig:622-681): non-finite -> 0,
// then clamp to [-100, 100].
inline float edge(float g) {
  if (!(g - g == 0.f)) g = 0.f;
  return g < -100.f ? -100.f : (g > 100.f ? 100.f : g);
}

template <typename R>
struct RowLse {
  R max, sum, lse;
};

// Reference op order: m = reduce max; s = x - m; e = exp(s); S = reduce add(e)
// (sequential); lse = m + log(S)  (qwen_test.mlir:257-264).
template <typename R>
RowLse<R> row_lse(const void* p, int dt, int64_t base, int64_t V) {
  R m = -INFINITY;
  for (int64_t v = 0; v < V; ++v) {
    const R x = static_cast<R>(loadd(p, dt, base + v));
    if (x > m) m = x;
  }
  R S = 0;
  for (int64_t v = 0; v < V; ++v) S += std::exp(static_cast<R>(loadd(p, dt, base + v)) - m);
  return {m, S, m + std::log(S)};
}

}  // namespace

extern "C" {

typedef struct oracle_rows_args {
  int64_t nrows, vocab;
  int32_t dtype;             // 0 f16, 1 bf16, 2 f32, 3 f64 (pcp_dtype codes)
  const void* logits;        // [nrows, V]
  const void* ref_logits;    // [nrows, V] or NULL
  const int64_t* ids;        // [nrows]; -100 = ignore
  const float* w;            // [nrows] mask weight
  const float* adv;          // [nrows] advantage of the row's sequence
  const float* seq_len;      // [nrows] max(sum mask, 1) of the row's sequence
  const float* old_logp;     // [nrows] or NULL (on-policy)
  float loss_norm;           // number of sequences averaged over
  int32_t loss_mode;         // 0 REINFORCE, 1 CLIP_KL
  float clip_eps, kl_beta;
  int32_t precision;         // 0 exact f64, 1 fp32 reference op order, 2 fp32 reference AD (REINFORCE)
  int32_t nthreads;          // <= 0: OpenMP default
  double* lp;                // outputs, each optional
  double* lr;
  double* token_loss;        // w * l'  (l' = -lp for REINFORCE, l for CLIP_KL)
  double* coef;              // d loss / d lp
  float* dlogits;            // [nrows, V]
} oracle_rows_args;

uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16(f); }
float oracle_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }
float oracle_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

void oracle_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(in[i]);
}

// rl_shepherd.zig:466-478, operation for operation in f32 (this file is built
// with -ffp-contract=off, so (r-mean)*(r-mean) and the sums round separately).
void oracle_advantages(const float* r, int64_t n, int64_t group, float eps, float* adv) {
  for (int64_t i = 0; i < n; i += group) {
    const int64_t e = (i + group < n) ? i + group : n;
    const float cnt = static_cast<float>(e - i);
    float sum = 0.f;
    for (int64_t k = i; k < e; ++k) sum += r[k];
    const float mean = sum / cnt;
    float ssd = 0.f;
    for (int64_t k = i; k < e; ++k) ssd += (r[k] - mean) * (r[k] - mean);
    const float sd = std::sqrt(ssd / cnt) + eps;
    for (int64_t k = i; k < e; ++k) adv[k] = (r[k] - mean) / sd;
  }
}

// Per-row log-prob: lp = x_y - lse (export_qwen_forward.py:156 returns -lp).
// precision 0: double; otherwise float in the reference op order.
void oracle_logprob(const void* logits, int32_t dtype, int64_t nrows, int64_t vocab, const int64_t* ids,
                    int32_t precision, int32_t nthreads, double* lp, double* lse) {
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t n = 0; n < nrows; ++n) {
    const int64_t base = n * vocab;
    const int64_t id = ids[n];
    double l, x;
    if (precision == kExact) {
      const RowLse<double> r = row_lse<double>(logits, dtype, base, vocab);
      l = r.lse;
      x = (id >= 0 && id < vocab) ? loadd(logits, dtype, base + id) : 0.0;
      if (lp) lp[n] = (id >= 0 && id < vocab) ? x - l : 0.0;
    } else {
      const RowLse<float> r = row_lse<float>(logits, dtype, base, vocab);
      l = r.lse;
      // lsm = (x - m) - log(S), then gather (qwen_test.mlir:260-275)
      const float s = (id >= 0 && id < vocab) ? load(logits, dtype, base + id) - r.max : 0.f;
      if (lp) lp[n] = (id >= 0 && id < vocab) ? static_cast<double>(s - std::log(r.sum)) : 0.0;
    }
    if (lse) lse[n] = l;
  }
}

// Loss terms and dlogits of a set of rows.
int oracle_grpo_rows(const oracle_rows_args* a) {
  if (!a || a->nrows < 0 || a->vocab < 1 || !a->logits || !a->ids || !a->w || !a->adv || !a->seq_len) return -1;
  if (a->loss_mode == kClipKl && !a->ref_logits) return -1;
  if (a->precision == kFaithful && a->loss_mode != kReinforce) return -1;
  if (a->nthreads > 0) omp_set_num_threads(a->nthreads);
  const int64_t V = a->vocab;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t n = 0; n < a->nrows; ++n) {
    const int64_t base = n * V;
    const int64_t id = a->ids[n];
    const bool live = a->w[n] != 0.f && id >= 0 && id < V;
    float* d = a->dlogits ? a->dlogits + base : nullptr;
    if (!live) {
      if (a->lp) a->lp[n] = 0.0;
      if (a->lr) a->lr[n] = 0.0;
      if (a->token_loss) a->token_loss[n] = 0.0;
      if (a->coef) a->coef[n] = 0.0;
      if (d) std::memset(d, 0, sizeof(float) * V);
      continue;
    }
    const double w = a->w[n], A = a->adv[n], L = a->seq_len[n], G = a->loss_norm;
    if (a->precision == kExact) {
      const RowLse<double> p = row_lse<double>(a->logits, a->dtype, base, V);
      const double lp = loadd(a->logits, a->dtype, base + id) - p.lse;
      double lr = 0.0;
      if (a->ref_logits) {
        const RowLse<double> q = row_lse<double>(a->ref_logits, a->dtype, base, V);
        lr = loadd(a->ref_logits, a->dtype, base + id) - q.lse;
      }
      double tl, c;
      const double scale = w / (G * L);
      if (a->loss_mode == kReinforce) {
        tl = w * (-lp);
        c = -A * scale;
      } else {
        const double old = a->old_logp ? static_cast<double>(a->old_logp[n]) : lp;
        const double rho = std::exp(lp - old);
        const double lo = 1.0 - a->clip_eps, hi = 1.0 + a->clip_eps;
        const double rc = rho < lo ? lo : (rho > hi ? hi : rho);
        const double surr = std::fmin(rho * A, rc * A);
        const double dlr = lr - lp, e = std::exp(dlr);
        tl = w * (-surr + a->kl_beta * (e - dlr - 1.0));
        const bool unclipped = (A >= 0.0) ? (rho <= hi) : (rho >= lo);
        c = scale * ((unclipped ? -A * rho : 0.0) + a->kl_beta * (1.0 - e));
      }
      if (a->lp) a->lp[n] = lp;
      if (a->lr) a->lr[n] = lr;
      if (a->token_loss) a->token_loss[n] = tl;
      if (a->coef) a->coef[n] = c;
      if (d) {
        for (int64_t v = 0; v < V; ++v) {
          const double sm = std::exp(loadd(a->logits, a->dtype, base + v) - p.lse);
          d[v] = static_cast<float>(c * ((v == id ? 1.0 : 0.0) - sm));
        }
      }
      continue;
    }

    // fp32 in the reference op order.
    const RowLse<float> p = row_lse<float>(a->logits, a->dtype, base, V);
    const float logS = std::log(p.sum);
    const float lpf = (load(a->logits, a->dtype, base + id) - p.max) - logS;
    float lrf = 0.f;
    if (a->ref_logits) {
      const RowLse<float> q = row_lse<float>(a->ref_logits, a->dtype, base, V);
      lrf = (load(a->ref_logits, a->dtype, base + id) - q.max) - std::log(q.sum);
    }
    const float wf = a->w[n], Af = a->adv[n], Lf = a->seq_len[n], Gf = a->loss_norm;
    float tl, c;
    if (a->precision == kFaithful) {
      // Reverse pass of mean -> *adv -> /seq_len -> sum_t -> *mask -> -lp with
      // the divideVJP guards: d weighted = 1/(G+1e-4); d seq_nll = that * adv;
      // d tok_sum = d seq_nll / (L + 1e-4); d tok = d tok_sum * mask; d lp = -d tok.
      const float d_weighted = edge(1.f / (Gf + 1e-4f));
      const float d_seq = edge(d_weighted * Af);
      const float d_tok = edge(edge(d_seq / (Lf + 1e-4f)) * wf);
      c = edge(-d_tok);
      tl = wf * (-lpf);
    } else {
      const float scale = wf / (Gf * Lf);
      if (a->loss_mode == kReinforce) {
        tl = wf * (-lpf);
        c = -Af * scale;
      } else {
        const float old = a->old_logp ? a->old_logp[n] : lpf;
        const float rho = std::exp(lpf - old);
        const float lo = 1.f - a->clip_eps, hi = 1.f + a->clip_eps;
        const float rc = std::fmin(std::fmax(rho, lo), hi);
        const float surr = std::fmin(rho * Af, rc * Af);
        const float dlr = lrf - lpf, e = std::exp(dlr);
        tl = wf * (-surr + a->kl_beta * (e - dlr - 1.f));
        const bool unclipped = (Af >= 0.f) ? (rho <= hi) : (rho >= lo);
        c = scale * ((unclipped ? -Af * rho : 0.f) + a->kl_beta * (1.f - e));
      }
    }
    if (a->lp) a->lp[n] = lpf;
    if (a->lr) a->lr[n] = lrf;
    if (a->token_loss) a->token_loss[n] = tl;
    if (a->coef) a->coef[n] = c;
    if (!d) continue;
    if (a->precision == kFaithful) {
      // d lsm = onehot * c; d logS = -c; d S = d logS / (S + 1e-4);
      // d s = d lsm + d S * exp(s); d m = -sum_v d s; d x = d s + [x == m] * d m.
      const float dS = edge(edge(-c) / (p.sum + 1e-4f));
      float sum_ds = 0.f;
      for (int64_t v = 0; v < V; ++v) {
        const float s = load(a->logits, a->dtype, base + v) - p.max;
        const float ds = (v == id ? edge(c) : 0.f) + edge(dS * std::exp(s));
        d[v] = ds;
        sum_ds += ds;
      }
      const float dm = edge(-sum_ds);
      for (int64_t v = 0; v < V; ++v) {
        const float x = load(a->logits, a->dtype, base + v);
        d[v] = edge(d[v] + (x == p.max ? dm : 0.f));
      }
    } else {
      for (int64_t v = 0; v < V; ++v) {
        const float sm = std::exp((load(a->logits, a->dtype, base + v) - p.max) - logS);
        d[v] = c * ((v == id ? 1.f : 0.f) - sm);
      }
    }
  }
  return 0;
}

// Element-wise check of a device's dlogits rows against the exact (float64) rows
// c * (onehot - softmax) of kExact above, without materialising the exact rows: per
// row the log-sum-exp is recomputed in double, then every element's error against the
// bar  tol = rel * |d| + kfloor * floor[n] + sub  is reduced to per-row statistics.
typedef struct oracle_check_args {
  int64_t nrows, vocab;
  int32_t dtype;             // logits storage (pcp_dtype codes 0..3)
  const void* logits;        // [nrows, V]
  const int64_t* ids;        // [nrows] targets (live rows only: 0 <= id < V)
  const double* coef;        // [nrows] exact coefficient d loss / d lp (oracle_grpo_rows, kExact)
  const double* floor_row;   // [nrows] absolute error floor of the row
  int32_t got_dtype;         // the device's dlogits: 0 f16, 1 bf16, 2 f32
  const void* got;           // [nrows, V]
  double rel, kfloor, sub;   // the bar's relative, floor and absolute terms
  double rel_min;            // max_rel counts elements with |d| >= rel_min * |coef|
  int32_t nthreads;
  double* max_usage;         // [nrows] max err / tol
  double* max_abs;           // [nrows] max err
  double* max_rel;           // [nrows] max err / |d| over |d| >= rel_min * |coef| (0 if none)
  int64_t* n_bad;            // [nrows] elements with err > tol
} oracle_check_args;

int oracle_check_dlogits(const oracle_check_args* a) {
  if (!a || a->nrows < 0 || a->vocab < 1 || !a->logits || !a->ids || !a->coef || !a->floor_row || !a->got ||
      !a->max_usage || !a->max_abs || !a->max_rel || !a->n_bad)
    return -1;
  if (a->got_dtype != kF16 && a->got_dtype != kBF16 && a->got_dtype != kF32) return -1;
  if (a->nthreads > 0) omp_set_num_threads(a->nthreads);
  const int64_t V = a->vocab;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t n = 0; n < a->nrows; ++n) {
    const int64_t base = n * V, id = a->ids[n];
    const RowLse<double> p = row_lse<double>(a->logits, a->dtype, base, V);
    const double c = a->coef[n], fl = a->kfloor * a->floor_row[n] + a->sub, thr = a->rel_min * std::fabs(c);
    double mu = 0.0, ma = 0.0, mr = 0.0;
    int64_t bad = 0;
    for (int64_t v = 0; v < V; ++v) {
      const double d = c * ((v == id ? 1.0 : 0.0) - std::exp(loadd(a->logits, a->dtype, base + v) - p.lse));
      const double g = loadd(a->got, a->got_dtype, base + v);
      const double err = std::fabs(g - d), ad = std::fabs(d);
      const double tol = a->rel * ad + fl;
      if (!(err <= tol)) ++bad;
      const double u = tol > 0.0 ? err / tol : (err > 0.0 ? INFINITY : 0.0);
      if (!(u <= mu)) mu = u;
      if (!(err <= ma)) ma = err;
      if (ad > 0.0 && ad >= thr && !(err / ad <= mr)) mr = err / ad;
    }
    a->max_usage[n] = mu;
    a->max_abs[n] = ma;
    a->max_rel[n] = mr;
    a->n_bad[n] = bad;
  }
  return 0;
}

int oracle_max_threads(void) { return omp_get_max_threads(); }

}  // extern "C"
