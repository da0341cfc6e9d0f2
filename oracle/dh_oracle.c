/*
 * dh_oracle.c — TEST INFRASTRUCTURE ONLY. Float64 CPU restatement of the reference's mixer
 * arithmetic, used by tests/, __graft_entry__.smoke() and bench.py's CPU baseline as the checker of
 * the HIP kernels. Nothing in the product links or calls this.
 *
 * Every array is a dense row-major double array; index arithmetic is spelled out in full.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static double sigm(double x) { return 1.0 / (1.0 + exp(-x)); }

/* Ring layout, reference dispatcher_hybrid/decoding.py:59-66 and fused_step.py:81-86:
 * ring j starts at 2^(j+1)-2 and has 2^(j+1) slots; position p sits at start + (p mod 2^(j+1)). */
int64_t dh_oracle_ring_offset(int j) { return ((int64_t)1 << (j + 1)) - 2; }
int64_t dh_oracle_ring_slot(int j, int64_t p) {
  return dh_oracle_ring_offset(j) + (p & (((int64_t)1 << (j + 1)) - 1));
}

/* Whether level l's edge into (b, t) is open: t >= 2^l and, with a doc mask, mask[b,t,l] > 0.
 * reference modeling_dispatcher.py:282-297 (level mask) and :311-323 (doc-reset mask). */
static int edge_open(const double* mask, int mask_L, int b, int T, int t, int l) {
  if (t < (1 << l)) return 0;
  if (!mask) return 1;
  return mask[((size_t)b * T + t) * mask_L + l] > 0.0;
}

/*
 * Gate pre-activations, reference modeling_dispatcher.py:100-109 (eager definition) and
 * fused_gates.py:38-93 (fused op):
 *   pre_x[b,t,l,h] = sum_g relu(A[b,t,g] + open * B[b,t-2^l,g])^2 * W_x[l,h,g] + b_x[l,h]
 * A, B: (nb, T, GH); W_x: (L, H, GH); b_x: (L, H); mask: (nb, T, mask_L) or NULL;
 * out_x: (nb, T, n_lv, H).
 */
void dh_oracle_gate_preacts(const double* A, const double* B, const double* Wi, const double* Wf,
                            const double* Wr, const double* bi, const double* bf, const double* br,
                            const double* mask, int mask_L, double* oi, double* of, double* orr,
                            int nb, int T, int GH, int H, int L, int n_lv) {
  (void)L;
  for (int b = 0; b < nb; ++b)
    for (int t = 0; t < T; ++t)
      for (int l = 0; l < n_lv; ++l) {
        const int open = edge_open(mask, mask_L, b, T, t, l);
        const double* a = A + ((size_t)b * T + t) * GH;
        const double* s = open ? B + ((size_t)b * T + (t - (1 << l))) * GH : NULL;
        for (int h = 0; h < H; ++h) {
          const double* wi = Wi + ((size_t)l * H + h) * GH;
          const double* wf = Wf + ((size_t)l * H + h) * GH;
          const double* wr = Wr + ((size_t)l * H + h) * GH;
          double si = 0, sf = 0, sr = 0;
          for (int g = 0; g < GH; ++g) {
            double x = a[g] + (s ? s[g] : 0.0);
            x = x > 0 ? x * x : 0.0;
            si += x * wi[g];
            sf += x * wf[g];
            sr += x * wr[g];
          }
          const size_t o = (((size_t)b * T + t) * n_lv + l) * H + h;
          oi[o] = si + bi[l * H + h];
          of[o] = sf + bf[l * H + h];
          orr[o] = sr + br[l * H + h];
        }
      }
}

/*
 * Level scan, reference modeling_dispatcher.py:86-88 and :111-121:
 *   a = sigmoid(pre_i)*M, f = sigmoid(pre_f)*M + (1-M), r = sigmoid(pre_r), M = edge_open
 *   for l < n_lv: V_new[t] = f[t,l] * V[t] + a[t,l] * r[t-2^l,l] * V[t-2^l]
 * pre_x: (nb, T, n_lv, H); V0, V: (nb, T, H*hd) with head h at columns [h*hd, (h+1)*hd);
 * scratch: nb*T*H*hd doubles.
 */
void dh_oracle_level_scan(const double* pi, const double* pf, const double* pr, const double* mask,
                          int mask_L, const double* V0, double* V, double* scratch, int nb, int T,
                          int H, int hd, int n_lv) {
  const size_t d = (size_t)H * hd;
  memcpy(V, V0, sizeof(double) * nb * T * d);
  for (int l = 0; l < n_lv; ++l) {
    memcpy(scratch, V, sizeof(double) * nb * T * d); /* previous level's state */
    for (int b = 0; b < nb; ++b)
      for (int t = 0; t < T; ++t) {
        if (!edge_open(mask, mask_L, b, T, t, l)) continue; /* f = 1, a = 0 */
        const int s = t - (1 << l);
        for (int h = 0; h < H; ++h) {
          const size_t gd = (((size_t)b * T + t) * n_lv + l) * H + h;
          const size_t gs = (((size_t)b * T + s) * n_lv + l) * H + h;
          const double a = sigm(pi[gd]), f = sigm(pf[gd]), r = sigm(pr[gs]);
          for (int e = 0; e < hd; ++e) {
            const size_t c = (size_t)h * hd + e;
            V[((size_t)b * T + t) * d + c] =
                f * scratch[((size_t)b * T + t) * d + c] + a * r * scratch[((size_t)b * T + s) * d + c];
          }
        }
      }
  }
}

/*
 * One decode step of a tree layer at position t, reference fused_step.py:26-88 and
 * decoding.py:187-222 (wrap mask only):
 *   for l < L: src = t - 2^l, ok = src >= 0
 *     hid = relu(A + ok * B_hist[src])^2 ; i,f,r as in the gate readout, i *= ok, f = f*ok + 1-ok
 *     rg_hist[t, l] = r
 *   V = V0 ; ring_0[slot(0,t)] = V0
 *   for l < L: V = f_l V + i_l ok rg_hist[src, l] ring_l[slot(l, src)] ;
 *              if l+1 < L: ring_{l+1}[slot(l+1, t)] = V
 *   Y = V
 * A: (nb, GH); B_hist: (nb, Tmax, GH); W_x: (L, H, GH); b_x: (L, H); rg_hist: (nb, Tmax, L, H);
 * V_ring: (nb, S, H*hd); V0, Y: (nb, H*hd).
 */
void dh_oracle_decode_step(const double* A, const double* B_hist, const double* Wi, const double* Wf,
                           const double* Wr, const double* bi, const double* bf, const double* br,
                           int64_t t, double* rg_hist, double* V_ring, const double* V0, double* Y,
                           int nb, int Tmax, int S, int GH, int H, int hd, int L) {
  const size_t d = (size_t)H * hd;
  double ig[16 * 64], fg[16 * 64];
  if (H > 64 || L > 16) return;
  for (int b = 0; b < nb; ++b) {
    for (int l = 0; l < L; ++l) {
      const int64_t src = t - ((int64_t)1 << l);
      const int ok = src >= 0;
      const double* a = A + (size_t)b * GH;
      const double* s = ok ? B_hist + ((size_t)b * Tmax + src) * GH : NULL;
      for (int h = 0; h < H; ++h) {
        double si = 0, sf = 0, sr = 0;
        for (int g = 0; g < GH; ++g) {
          double x = a[g] + (s ? s[g] : 0.0);
          x = x > 0 ? x * x : 0.0;
          si += x * Wi[((size_t)l * H + h) * GH + g];
          sf += x * Wf[((size_t)l * H + h) * GH + g];
          sr += x * Wr[((size_t)l * H + h) * GH + g];
        }
        ig[l * H + h] = ok ? sigm(si + bi[l * H + h]) : 0.0;
        fg[l * H + h] = ok ? sigm(sf + bf[l * H + h]) : 1.0;
        rg_hist[(((size_t)b * Tmax + t) * L + l) * H + h] = sigm(sr + br[l * H + h]);
      }
    }
    double* ring = V_ring + (size_t)b * S * d;
    for (int h = 0; h < H; ++h)
      for (int e = 0; e < hd; ++e) {
        const size_t c = (size_t)h * hd + e;
        double v = V0[(size_t)b * d + c];
        ring[dh_oracle_ring_slot(0, t) * d + c] = v;
        for (int l = 0; l < L; ++l) {
          const int64_t src = t - ((int64_t)1 << l);
          double msg = 0.0;
          if (src >= 0)
            msg = rg_hist[(((size_t)b * Tmax + src) * L + l) * H + h] * ring[dh_oracle_ring_slot(l, src) * d + c];
          v = fg[l * H + h] * v + ig[l * H + h] * msg;
          if (l + 1 < L) ring[dh_oracle_ring_slot(l + 1, t) * d + c] = v;
        }
        Y[(size_t)b * d + c] = v;
      }
  }
}
