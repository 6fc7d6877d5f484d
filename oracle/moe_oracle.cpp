// MoE layer CPU oracle -- TEST INFRASTRUCTURE ONLY.
//
// This file restates, on the CPU, the arithmetic of oxidizr's Mixture-of-
// Experts layer (forward and every gradient) so that the HIP implementation in
// oxidizr_amd/ can be checked against it. Only tests/, __graft_entry__.smoke()
// and bench.py's cpu_baseline leg may load it, and only as the checker or the
// timed CPU baseline. The product library never links or calls it.
//
// Where the semantics come from (reference = /root/reference, ml-rust/oxidizr):
//   * layer shape contract, flatten [B,S,H] -> [T,H]:      src/model.rs:1834-1885
//   * router gate = Linear [E,H], no bias by default:       src/model.rs:1575-1630, 1506-1537
//   * softmax then top-k routing:                            docs/architecture/moe.md:149-153
//   * router config (temperature, SwitchPlusSquaredProb):   src/model.rs:1899-1909
//   * SwiGLU expert down(silu(gate x) * up x):               src/model.rs:1284-1290
//   * expert weights gate/up [I,H], down [H,I]:              src/model.rs:1422-1445
//   * optional shared expert scaled by s(k):                 src/model.rs:1674-1702, 1923-1925
//   * returns (out, aux_loss, z_loss):                       src/model.rs:1830-1833, 1884
//   * experts that see no token get no gradient entry:       src/trainer.rs:556-566
// The arithmetic itself lives in boostr 0.10.0 (boostr::nn::moe), which is not
// vendored in the reference and cannot be fetched. Its constants are therefore
// plan parameters here, with these defaults: temperature 1, no top-k
// renormalisation, aux = E*(c_sw*sum_e f_e P_e + c_sq*sum_e P_e^2) with unit
// coefficients, z = mean_t lse_t^2, shared-expert scale 1, lowest-index tie-break.
//
// Every function is deterministic (fixed summation order, OpenMP only across
// independent output rows), in two precisions: double (the checker) and float
// (the timed CPU baseline).
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>
#include <algorithm>
#include <string>
#include <omp.h>

extern "C" {
typedef struct {
  int32_t T, H, E, k, I, S;
  int32_t norm_topk;   // renormalise the k selected probabilities to sum 1
  int32_t has_bias;    // router Linear carries a bias [E]
  double tau;          // router temperature: probs = softmax(logits / tau)
  double shared_scale; // out += shared_scale * shared_expert(x)
  double aux_switch;   // coefficient of the Switch term E*sum f_e P_e
  double aux_sqprob;   // coefficient of the squared-probability term E*sum P_e^2
} oracle_cfg;
}

namespace {

template <typename R>
inline R silu(R g) { return g / (R(1) + std::exp(-g)); }

template <typename R>
inline R dsilu(R g) {  // d/dg [g * sigmoid(g)]
  R s = R(1) / (R(1) + std::exp(-g));
  return s * (R(1) + g * (R(1) - s));
}

// C[m, n] = sum_k A[m, k] * B[n, k]; A is [M, K], B is [N, K], both row-major.
// Fixed summation order: 8 interleaved partial sums over k, then summed in order.
template <typename R>
void gemm_nt(int M, int N, int K, const R* A, int lda, const R* B, int ldb, R* C, int ldc) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int n = 0; n < N; ++n) {
      const R* a = A + (size_t)m * lda;
      const R* b = B + (size_t)n * ldb;
      R acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      int k = 0;
      for (; k + 8 <= K; k += 8)
        for (int u = 0; u < 8; ++u) acc[u] += a[k + u] * b[k + u];
      for (; k < K; ++k) acc[0] += a[k] * b[k];
      R s = 0;
      for (int u = 0; u < 8; ++u) s += acc[u];
      C[(size_t)m * ldc + n] = s;
    }
  }
}

// C[m, n] = sum_k A[m, k] * B[k, n]; A is [M, K], B is [K, N]. k ascending.
// Parallel over rows and 256-wide column blocks.
template <typename R>
void gemm_nn(int M, int N, int K, const R* A, int lda, const R* B, int ldb, R* C, int ldc) {
  const int NB = (N + 255) / 256;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int nb = 0; nb < NB; ++nb) {
      const int n0 = nb * 256, n1 = std::min(N, n0 + 256);
      R* c = C + (size_t)m * ldc;
      for (int n = n0; n < n1; ++n) c[n] = 0;
      for (int k = 0; k < K; ++k) {
        R a = A[(size_t)m * lda + k];
        const R* b = B + (size_t)k * ldb;
        for (int n = n0; n < n1; ++n) c[n] += a * b[n];
      }
    }
  }
}

// C[m, n] = sum_k A[k, m] * B[k, n]; A is [K, M], B is [K, N]. k ascending.
// Parallel over rows and 256-wide column blocks.
template <typename R>
void gemm_tn(int M, int N, int K, const R* A, int lda, const R* B, int ldb, R* C, int ldc) {
  const int NB = (N + 255) / 256;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int nb = 0; nb < NB; ++nb) {
      const int n0 = nb * 256, n1 = std::min(N, n0 + 256);
      R* c = C + (size_t)m * ldc;
      for (int n = n0; n < n1; ++n) c[n] = 0;
      for (int k = 0; k < K; ++k) {
        R a = A[(size_t)k * lda + m];
        const R* b = B + (size_t)k * ldb;
        for (int n = n0; n < n1; ++n) c[n] += a * b[n];
      }
    }
  }
}

// Softmax over logits/tau, log-sum-exp, and top-k on the raw logits with the
// lowest expert index winning ties; slot 0 holds the largest logit.
template <typename R>
void route_rows(const oracle_cfg& c, int T, const R* logits, R* probs, R* lse,
                int32_t* idx, R* w) {
  const int E = c.E, k = c.k;
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    const R* l = logits + (size_t)t * E;
    R mx = l[0] / R(c.tau);
    for (int e = 1; e < E; ++e) mx = std::max(mx, l[e] / R(c.tau));
    R den = 0;
    for (int e = 0; e < E; ++e) den += std::exp(l[e] / R(c.tau) - mx);
    for (int e = 0; e < E; ++e) probs[(size_t)t * E + e] = std::exp(l[e] / R(c.tau) - mx) / den;
    lse[t] = mx + std::log(den);
    std::vector<char> taken(E, 0);
    R wsum = 0;
    for (int j = 0; j < k; ++j) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || l[e] > l[best]) best = e;  // strict '>' keeps the lower index on ties
      }
      taken[best] = 1;
      idx[(size_t)t * k + j] = best;
      w[(size_t)t * k + j] = probs[(size_t)t * E + best];
      wsum += w[(size_t)t * k + j];
    }
    if (c.norm_topk)
      for (int j = 0; j < k; ++j) w[(size_t)t * k + j] /= wsum;
  }
}

// Stable counting sort of the T*k assignments by expert: canonical order is
// expert ascending, then token ascending. perm[pos] = t*k + j; inv_perm inverts it.
void dispatch_rows(int T, int k, int E, const int32_t* idx, int32_t* counts,
                   int32_t* offsets, int32_t* perm, int32_t* inv_perm) {
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int a = 0; a < T * k; ++a) counts[idx[a]]++;
  offsets[0] = 0;
  for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
  std::vector<int32_t> cursor(offsets, offsets + E);
  for (int t = 0; t < T; ++t)
    for (int j = 0; j < k; ++j) {
      int a = t * k + j;
      int pos = cursor[idx[a]]++;
      perm[pos] = a;
      inv_perm[a] = pos;
    }
}

template <typename R>
struct Oracle {
  oracle_cfg c;
  int T = 0;
  // inputs (borrowed from the caller between forward and backward)
  const R *x = nullptr, *wr = nullptr, *bias = nullptr, *wg = nullptr, *wu = nullptr,
          *wd = nullptr, *swg = nullptr, *swu = nullptr, *swd = nullptr;
  // forward state
  std::vector<R> logits, probs, lse, topw, xp, G, U, A, Y, sG, sU, sA, sY;
  std::vector<int32_t> topi, counts, offsets, perm, inv_perm;
  R aux = 0, z = 0;

  explicit Oracle(const oracle_cfg& cfg) : c(cfg) {}

  void forward(int T_, const R* x_, const R* wr_, const R* bias_, const R* wg_, const R* wu_,
               const R* wd_, const R* swg_, const R* swu_, const R* swd_,
               const float* logits_in, R* out) {
    T = T_;
    x = x_; wr = wr_; bias = bias_; wg = wg_; wu = wu_; wd = wd_; swg = swg_; swu = swu_; swd = swd_;
    const int H = c.H, E = c.E, k = c.k, I = c.I, S = c.S;
    const size_t TK = (size_t)T * k;
    logits.assign((size_t)T * E, 0);
    if (logits_in) {
      for (size_t i = 0; i < logits.size(); ++i) logits[i] = R(logits_in[i]);
    } else {
      gemm_nt<R>(T, E, H, x, H, wr, H, logits.data(), E);
      if (c.has_bias && bias)
        for (int t = 0; t < T; ++t)
          for (int e = 0; e < E; ++e) logits[(size_t)t * E + e] += bias[e];
    }
    probs.assign((size_t)T * E, 0);
    lse.assign(T, 0);
    topi.assign(TK, 0);
    topw.assign(TK, 0);
    route_rows<R>(c, T, logits.data(), probs.data(), lse.data(), topi.data(), topw.data());
    counts.assign(E, 0);
    offsets.assign(E + 1, 0);
    perm.assign(TK, 0);
    inv_perm.assign(TK, 0);
    dispatch_rows(T, k, E, topi.data(), counts.data(), offsets.data(), perm.data(), inv_perm.data());

    // gather rows of x into expert order
    xp.assign(TK * H, 0);
    for (size_t p = 0; p < TK; ++p)
      std::memcpy(&xp[p * H], x + (size_t)(perm[p] / k) * H, sizeof(R) * H);
    G.assign(TK * I, 0);
    U.assign(TK * I, 0);
    A.assign(TK * I, 0);
    Y.assign(TK * H, 0);
    for (int e = 0; e < E; ++e) {
      int M = counts[e];
      if (M == 0) continue;
      size_t r0 = offsets[e];
      gemm_nt<R>(M, I, H, &xp[r0 * H], H, wg + (size_t)e * I * H, H, &G[r0 * I], I);
      gemm_nt<R>(M, I, H, &xp[r0 * H], H, wu + (size_t)e * I * H, H, &U[r0 * I], I);
      for (size_t q = r0 * I; q < (r0 + M) * I; ++q) A[q] = silu(G[q]) * U[q];
      gemm_nt<R>(M, H, I, &A[r0 * I], I, wd + (size_t)e * H * I, I, &Y[r0 * H], H);
    }
    if (S > 0) {
      sG.assign((size_t)T * S, 0);
      sU.assign((size_t)T * S, 0);
      sA.assign((size_t)T * S, 0);
      sY.assign((size_t)T * H, 0);
      gemm_nt<R>(T, S, H, x, H, swg, H, sG.data(), S);
      gemm_nt<R>(T, S, H, x, H, swu, H, sU.data(), S);
      for (size_t q = 0; q < sA.size(); ++q) sA[q] = silu(sG[q]) * sU[q];
      gemm_nt<R>(T, H, S, sA.data(), S, swd, S, sY.data(), H);
    }
    // weighted combine in fixed slot order, then the scaled shared expert
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
      for (int h = 0; h < H; ++h) {
        R acc = 0;
        for (int j = 0; j < k; ++j)
          acc += topw[(size_t)t * k + j] * Y[(size_t)inv_perm[(size_t)t * k + j] * H + h];
        if (S > 0) acc += R(c.shared_scale) * sY[(size_t)t * H + h];
        out[(size_t)t * H + h] = acc;
      }
    }
    // load-balance loss: f_e = M_e / (T k), P_e = mean_t probs[t, e]
    R sw = 0, sq = 0;
    for (int e = 0; e < E; ++e) {
      R P = 0;
      for (int t = 0; t < T; ++t) P += probs[(size_t)t * E + e];
      P /= R(T);
      R f = R(counts[e]) / R(TK);
      sw += f * P;
      sq += P * P;
    }
    aux = R(E) * (R(c.aux_switch) * sw + R(c.aux_sqprob) * sq);
    R zz = 0;
    for (int t = 0; t < T; ++t) zz += lse[t] * lse[t];
    z = zz / R(T);
  }

  void backward(const R* dout, R d_aux, R d_z, R* dx, R* dwr, R* dbias, R* dwg, R* dwu,
                R* dwd, R* dswg, R* dswu, R* dswd, uint8_t* has_grad) {
    const int H = c.H, E = c.E, k = c.k, I = c.I, S = c.S;
    const size_t TK = (size_t)T * k;
    // combine backward: d weight = <dout_t, Y_pos>, dY_pos = w * dout_t
    std::vector<R> dw(TK, 0), dY(TK * H, 0);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t)
      for (int j = 0; j < k; ++j) {
        size_t a = (size_t)t * k + j, pos = inv_perm[a];
        R s = 0;
        for (int h = 0; h < H; ++h) {
          s += dout[(size_t)t * H + h] * Y[pos * H + h];
          dY[pos * H + h] = topw[a] * dout[(size_t)t * H + h];
        }
        dw[a] = s;
      }
    // routed experts
    std::vector<R> dA(TK * I, 0), dG(TK * I, 0), dU(TK * I, 0), dXp(TK * H, 0), tmp;
    for (int e = 0; e < E; ++e) {
      int M = counts[e];
      has_grad[e] = M > 0;
      if (M == 0) continue;  // no gradient entry: buffers are left untouched
      size_t r0 = offsets[e];
      gemm_nn<R>(M, I, H, &dY[r0 * H], H, wd + (size_t)e * H * I, I, &dA[r0 * I], I);
      gemm_tn<R>(H, I, M, &dY[r0 * H], H, &A[r0 * I], I, dwd + (size_t)e * H * I, I);
      for (size_t q = r0 * I; q < (r0 + M) * I; ++q) {
        dG[q] = dA[q] * U[q] * dsilu(G[q]);
        dU[q] = dA[q] * silu(G[q]);
      }
      tmp.assign((size_t)M * H, 0);
      gemm_nn<R>(M, H, I, &dG[r0 * I], I, wg + (size_t)e * I * H, H, &dXp[r0 * H], H);
      gemm_nn<R>(M, H, I, &dU[r0 * I], I, wu + (size_t)e * I * H, H, tmp.data(), H);
      for (size_t q = 0; q < (size_t)M * H; ++q) dXp[r0 * H + q] += tmp[q];
      gemm_tn<R>(I, H, M, &dG[r0 * I], I, &xp[r0 * H], H, dwg + (size_t)e * I * H, H);
      gemm_tn<R>(I, H, M, &dU[r0 * I], I, &xp[r0 * H], H, dwu + (size_t)e * I * H, H);
    }
    // shared expert
    std::vector<R> dxs;
    if (S > 0) {
      std::vector<R> dYs((size_t)T * H), dAs((size_t)T * S), dGs((size_t)T * S), dUs((size_t)T * S);
      dxs.assign((size_t)T * H, 0);
      for (size_t q = 0; q < dYs.size(); ++q) dYs[q] = R(c.shared_scale) * dout[q];
      gemm_nn<R>(T, S, H, dYs.data(), H, swd, S, dAs.data(), S);
      gemm_tn<R>(H, S, T, dYs.data(), H, sA.data(), S, dswd, S);
      for (size_t q = 0; q < dAs.size(); ++q) {
        dGs[q] = dAs[q] * sU[q] * dsilu(sG[q]);
        dUs[q] = dAs[q] * silu(sG[q]);
      }
      tmp.assign((size_t)T * H, 0);
      gemm_nn<R>(T, H, S, dGs.data(), S, swg, H, dxs.data(), H);
      gemm_nn<R>(T, H, S, dUs.data(), S, swu, H, tmp.data(), H);
      for (size_t q = 0; q < dxs.size(); ++q) dxs[q] += tmp[q];
      gemm_tn<R>(S, H, T, dGs.data(), S, x, H, dswg, H);
      gemm_tn<R>(S, H, T, dUs.data(), S, x, H, dswu, H);
    }
    // router: d probs from the combine weights and the aux loss, then the
    // softmax Jacobian, plus the z-loss term; divided by tau for d logits.
    std::vector<R> coefP(E), dlog((size_t)T * E);
    for (int e = 0; e < E; ++e) {
      R P = 0;
      for (int t = 0; t < T; ++t) P += probs[(size_t)t * E + e];
      P /= R(T);
      R f = R(counts[e]) / R(TK);
      coefP[e] = d_aux * R(E) * (R(c.aux_switch) * f + R(2) * R(c.aux_sqprob) * P) / R(T);
    }
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
      std::vector<R> dp(E);
      for (int e = 0; e < E; ++e) dp[e] = coefP[e];
      if (c.norm_topk) {
        R psum = 0, dot = 0;
        for (int j = 0; j < k; ++j) psum += probs[(size_t)t * E + topi[(size_t)t * k + j]];
        for (int j = 0; j < k; ++j) dot += dw[(size_t)t * k + j] * topw[(size_t)t * k + j];
        for (int j = 0; j < k; ++j)
          dp[topi[(size_t)t * k + j]] += (dw[(size_t)t * k + j] - dot) / psum;
      } else {
        for (int j = 0; j < k; ++j) dp[topi[(size_t)t * k + j]] += dw[(size_t)t * k + j];
      }
      R dot = 0;
      for (int e = 0; e < E; ++e) dot += probs[(size_t)t * E + e] * dp[e];
      for (int e = 0; e < E; ++e) {
        R p = probs[(size_t)t * E + e];
        R ds = p * (dp[e] - dot) + d_z * R(2) / R(T) * lse[t] * p;
        dlog[(size_t)t * E + e] = ds / R(c.tau);
      }
    }
    if (dbias)
      for (int e = 0; e < E; ++e) {
        R s = 0;
        for (int t = 0; t < T; ++t) s += dlog[(size_t)t * E + e];
        dbias[e] = s;
      }
    gemm_tn<R>(E, H, T, dlog.data(), E, x, H, dwr, H);
    gemm_nn<R>(T, H, E, dlog.data(), E, wr, H, dx, H);
    // scatter back: dx_t += sum_j dXp[pos(t, j)] (fixed slot order) + shared
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t)
      for (int h = 0; h < H; ++h) {
        R acc = dx[(size_t)t * H + h];
        for (int j = 0; j < k; ++j) acc += dXp[(size_t)inv_perm[(size_t)t * k + j] * H + h];
        if (S > 0) acc += dxs[(size_t)t * H + h];
        dx[(size_t)t * H + h] = acc;
      }
  }
};

struct Handle {
  int precision;
  void* impl;
};

template <typename R>
int get_state(Oracle<R>* o, const char* name, void* dst) {
  auto cpy = [&](const auto& v) {
    std::memcpy(dst, v.data(), v.size() * sizeof(v[0]));
    return 0;
  };
  std::string n(name);
  if (n == "logits") return cpy(o->logits);
  if (n == "probs") return cpy(o->probs);
  if (n == "lse") return cpy(o->lse);
  if (n == "topk_idx") return cpy(o->topi);
  if (n == "topk_w") return cpy(o->topw);
  if (n == "counts") return cpy(o->counts);
  if (n == "offsets") return cpy(o->offsets);
  if (n == "perm") return cpy(o->perm);
  if (n == "inv_perm") return cpy(o->inv_perm);
  if (n == "x_perm") return cpy(o->xp);
  if (n == "G") return cpy(o->G);
  if (n == "U") return cpy(o->U);
  if (n == "A") return cpy(o->A);
  if (n == "Y") return cpy(o->Y);
  if (n == "shared_Y") return cpy(o->sY);
  if (n == "aux") { *(R*)dst = o->aux; return 0; }
  if (n == "z") { *(R*)dst = o->z; return 0; }
  return -1;
}

}  // namespace

extern "C" {

// precision: 64 (double arrays) or 32 (float arrays).
void* oracle_create(const oracle_cfg* cfg, int precision) {
  if (!cfg || (precision != 64 && precision != 32)) return nullptr;
  if (cfg->k < 1 || cfg->k > cfg->E || cfg->I <= 0 || cfg->H <= 0) return nullptr;
  Handle* h = new Handle{precision, nullptr};
  if (precision == 64) h->impl = new Oracle<double>(*cfg);
  else h->impl = new Oracle<float>(*cfg);
  return h;
}

void oracle_destroy(void* hp) {
  Handle* h = (Handle*)hp;
  if (!h) return;
  if (h->precision == 64) delete (Oracle<double>*)h->impl;
  else delete (Oracle<float>*)h->impl;
  delete h;
}

void oracle_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int oracle_max_threads(void) { return omp_get_max_threads(); }

// Forward. Arrays are of the handle's precision; weights are packed per
// expert: wg, wu [E, I, H]; wd [E, H, I]; shared swg, swu [S, H]; swd [H, S].
// logits_in (float [T, E], nullable) replaces the router GEMM so routing can be
// compared on identical logits.
int oracle_forward(void* hp, int T, const void* x, const void* wr, const void* bias,
                   const void* wg, const void* wu, const void* wd, const void* swg,
                   const void* swu, const void* swd, const float* logits_in, void* out) {
  Handle* h = (Handle*)hp;
  if (!h || T < 0) return -1;
  if (h->precision == 64)
    ((Oracle<double>*)h->impl)->forward(T, (const double*)x, (const double*)wr, (const double*)bias,
        (const double*)wg, (const double*)wu, (const double*)wd, (const double*)swg,
        (const double*)swu, (const double*)swd, logits_in, (double*)out);
  else
    ((Oracle<float>*)h->impl)->forward(T, (const float*)x, (const float*)wr, (const float*)bias,
        (const float*)wg, (const float*)wu, (const float*)wd, (const float*)swg,
        (const float*)swu, (const float*)swd, logits_in, (float*)out);
  return 0;
}

int oracle_backward(void* hp, const void* dout, double d_aux, double d_z, void* dx, void* dwr,
                    void* dbias, void* dwg, void* dwu, void* dwd, void* dswg, void* dswu,
                    void* dswd, uint8_t* has_grad) {
  Handle* h = (Handle*)hp;
  if (!h) return -1;
  if (h->precision == 64)
    ((Oracle<double>*)h->impl)->backward((const double*)dout, d_aux, d_z, (double*)dx,
        (double*)dwr, (double*)dbias, (double*)dwg, (double*)dwu, (double*)dwd, (double*)dswg,
        (double*)dswu, (double*)dswd, has_grad);
  else
    ((Oracle<float>*)h->impl)->backward((const float*)dout, (float)d_aux, (float)d_z, (float*)dx,
        (float*)dwr, (float*)dbias, (float*)dwg, (float*)dwu, (float*)dwd, (float*)dswg,
        (float*)dswu, (float*)dswd, has_grad);
  return 0;
}

// Copy a named forward intermediate (see get_state) into dst.
int oracle_get(void* hp, const char* name, void* dst) {
  Handle* h = (Handle*)hp;
  if (!h) return -1;
  if (h->precision == 64) return get_state((Oracle<double>*)h->impl, name, dst);
  return get_state((Oracle<float>*)h->impl, name, dst);
}

// Stage entry points used to pin routing and dispatch on their own.
int oracle_route_f64(const oracle_cfg* cfg, int T, const double* logits, double* probs,
                     double* lse, int32_t* idx, double* w) {
  route_rows<double>(*cfg, T, logits, probs, lse, idx, w);
  return 0;
}

int oracle_dispatch(int T, int k, int E, const int32_t* idx, int32_t* counts, int32_t* offsets,
                    int32_t* perm, int32_t* inv_perm) {
  for (int a = 0; a < T * k; ++a)
    if (idx[a] < 0 || idx[a] >= E) return -2;
  dispatch_rows(T, k, E, idx, counts, offsets, perm, inv_perm);
  return 0;
}

}  // extern "C"
