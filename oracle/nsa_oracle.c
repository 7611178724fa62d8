/*
 * CPU ORACLE FOR TESTS ONLY.  This file is test infrastructure: it is compiled into
 * oracle/liboracle.so and used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker of the HIP path.  The product
 * (libnsa_hip.so and the nsa package) never links, loads or calls it.
 *
 * It restates, in plain C, the semantics of the reference's NSA hot path:
 *
 *   oracle_attn_fwd / oracle_attn_bwd   (double precision)
 *     sliding window   nsa/reference.py:13-78   (key j visible iff t-w < j <= t)
 *     compression      nsa/reference.py:81-147  (block_ends[i] <= t, empty row -> 0)
 *     selection        nsa/reference.py:205-254 (union of selected blocks, causal)
 *     backward: the reference kernels' algebra, nsa/kernels.py:1303-1530
 *       (p = exp(s - M - L), dS = p (dP - D), dQ = scale dS K, dK = scale dS^T Q).
 *
 *   oracle_score_topn   (fp32, fixed operation order)
 *     Eq. 8  nsa/kernels.py:2316-2343  p_cmp = softmax over visible compressed blocks
 *            of (q . K_cmp) * scale, block 0 made visible for rows with none
 *     Eq. 9  nsa/kernels.py:1920-1962  p_slc[j] = sum_{m<s} sum_{n<a} p_cmp[s*j+m+n]
 *     Eq. 10 nsa/kernels.py:1990-1993  sum over the group's heads
 *     top-n  nsa/kernels.py:1995-2040  stable descending sort (ties -> lower index),
 *            fixed blocks [0, max(0,(t-l')//l'), t//l'] merged in front, de-duplicated,
 *            truncated to n, padded with -1.
 *   The fp32 operation order is fixed here (and reproduced by the GPU kernel) so the
 *   selected indices can be compared bit for bit; see the comments at each step.
 *
 *   oracle_exp32: the exp() used by that pipeline (Cody-Waite reduction + degree-7
 *   Taylor polynomial, flushed to 0 below -64), written from the mathematics.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- exp ---- */
float oracle_exp32(float x) {
  const float kLog2e = 1.44269504088896341f;
  const float kLn2Hi = 0.693145751953125f;       /* ln2 rounded to 16 significant bits */
  const float kLn2Lo = 1.42860682030941723212e-6f; /* ln2 - kLn2Hi */
  if (!(x >= -64.0f)) return 0.0f;
  if (x > 0.0f) x = 0.0f; /* callers pass s - max <= 0 */
  float k = rintf(x * kLog2e);
  float r = fmaf(-k, kLn2Hi, x);
  r = fmaf(-k, kLn2Lo, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  union {
    uint32_t u;
    float f;
  } sc;
  sc.u = (uint32_t)((int)k + 127) << 23;
  return p * sc.f;
}

/* ------------------------------------------------------- attention ------ */
enum { ORACLE_SLIDING = 0, ORACLE_COMPRESSION = 1, ORACLE_SELECTION = 2 };

/* Visible keys of query t in group (b,g): writes the list to `keys`, returns count.
 * idx: [B,G,Tq,n] int64 (selection). */
static int visible_keys(int kind, int t, int Tkv, int window, const int32_t* block_ends, const int64_t* idxrow, int n,
                        int lprime, int causal, int* keys, unsigned char* mark) {
  int cnt = 0;
  if (kind == ORACLE_SLIDING) {
    int lo = t - window + 1;
    if (lo < 0) lo = 0;
    for (int j = lo; j <= t && j < Tkv; ++j) keys[cnt++] = j;
  } else if (kind == ORACLE_COMPRESSION) {
    for (int i = 0; i < Tkv; ++i)
      if (block_ends[i] <= t) keys[cnt++] = i;
  } else {
    memset(mark, 0, (size_t)Tkv);
    for (int s = 0; s < n; ++s) {
      int64_t blk = idxrow[s];
      if (blk < 0) continue;
      int64_t st = blk * lprime, en = st + lprime;
      if (en > Tkv) en = Tkv;
      for (int64_t j = st; j < en; ++j) mark[j] = 1;
    }
    for (int j = 0; j < Tkv; ++j)
      if (mark[j] && (!causal || j <= t)) keys[cnt++] = j;
  }
  return cnt;
}

/* q [B,H,Tq,dk], k [B,G,Tkv,dk], v [B,G,Tkv,dv] (row-major, double).
 * out [B,H,Tq,dv], L, M [B,H,Tq].  Empty rows: out 0, L = M = -inf. */
/* tmap (optional): row r of q / out is query position tmap[r] (idx rows are indexed
 * by r as well); NULL means row r is position r. */
int oracle_attn_fwd(int kind, int B, int H, int G, int Tq, int Tkv, int dk, int dv, const double* q, const double* k,
                    const double* v, double scale, int window, const int32_t* block_ends, const int64_t* idx, int n,
                    int lprime, int causal, const int32_t* tmap, double* out, double* L, double* M) {
  const int hpg = H / G;
  int* keys = (int*)malloc(sizeof(int) * (size_t)(Tkv > 0 ? Tkv : 1));
  unsigned char* mark = (unsigned char*)malloc((size_t)(Tkv > 0 ? Tkv : 1));
  double* s = (double*)malloc(sizeof(double) * (size_t)(Tkv > 0 ? Tkv : 1));
  if (!keys || !mark || !s) return 1;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int g = h / hpg;
      for (int tr = 0; tr < Tq; ++tr) {
        const int t = tmap ? tmap[tr] : tr;
        const int64_t* idxrow = idx ? idx + (((int64_t)b * G + g) * Tq + tr) * n : NULL;
        const int cnt = visible_keys(kind, t, Tkv, window, block_ends, idxrow, n, lprime, causal, keys, mark);
        const double* qr = q + (((int64_t)b * H + h) * Tq + tr) * dk;
        double* orow = out + (((int64_t)b * H + h) * Tq + tr) * dv;
        const int64_t r = ((int64_t)b * H + h) * Tq + tr;
        for (int e = 0; e < dv; ++e) orow[e] = 0.0;
        if (cnt == 0) {
          L[r] = -INFINITY;
          M[r] = -INFINITY;
          continue;
        }
        double mx = -INFINITY;
        for (int c = 0; c < cnt; ++c) {
          const double* kr = k + (((int64_t)b * G + g) * Tkv + keys[c]) * dk;
          double acc = 0.0;
          for (int d = 0; d < dk; ++d) acc += qr[d] * kr[d];
          s[c] = acc * scale;
          if (s[c] > mx) mx = s[c];
        }
        double l = 0.0;
        for (int c = 0; c < cnt; ++c) {
          const double p = exp(s[c] - mx);
          l += p;
          const double* vr = v + (((int64_t)b * G + g) * Tkv + keys[c]) * dv;
          for (int e = 0; e < dv; ++e) orow[e] += p * vr[e];
        }
        for (int e = 0; e < dv; ++e) orow[e] /= l;
        L[r] = log(l);
        M[r] = mx;
      }
    }
  free(keys);
  free(mark);
  free(s);
  return 0;
}

/* Backward with the forward's statistics recomputed in double (so the oracle's
 * gradients are those of its own forward).  dq overwritten, dk/dv [B,G,Tkv,*]
 * overwritten. */
int oracle_attn_bwd(int kind, int B, int H, int G, int Tq, int Tkv, int dk, int dv, const double* q, const double* k,
                    const double* v, const double* dout, double scale, int window, const int32_t* block_ends,
                    const int64_t* idx, int n, int lprime, int causal, const int32_t* tmap, double* dq, double* dkk,
                    double* dvv) {
  const int hpg = H / G;
  int* keys = (int*)malloc(sizeof(int) * (size_t)(Tkv > 0 ? Tkv : 1));
  unsigned char* mark = (unsigned char*)malloc((size_t)(Tkv > 0 ? Tkv : 1));
  double* p = (double*)malloc(sizeof(double) * (size_t)(Tkv > 0 ? Tkv : 1));
  double* o = (double*)malloc(sizeof(double) * (size_t)(dv > 0 ? dv : 1));
  if (!keys || !mark || !p || !o) return 1;
  memset(dkk, 0, sizeof(double) * (size_t)B * G * Tkv * dk);
  memset(dvv, 0, sizeof(double) * (size_t)B * G * Tkv * dv);
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int g = h / hpg;
      for (int tr = 0; tr < Tq; ++tr) {
        const int t = tmap ? tmap[tr] : tr;
        const int64_t* idxrow = idx ? idx + (((int64_t)b * G + g) * Tq + tr) * n : NULL;
        const int cnt = visible_keys(kind, t, Tkv, window, block_ends, idxrow, n, lprime, causal, keys, mark);
        const int64_t r = ((int64_t)b * H + h) * Tq + tr;
        const double* qr = q + r * dk;
        const double* dor = dout + r * dv;
        double* dqr = dq + r * dk;
        for (int d = 0; d < dk; ++d) dqr[d] = 0.0;
        if (cnt == 0) continue;
        double mx = -INFINITY;
        for (int c = 0; c < cnt; ++c) {
          const double* kr = k + (((int64_t)b * G + g) * Tkv + keys[c]) * dk;
          double acc = 0.0;
          for (int d = 0; d < dk; ++d) acc += qr[d] * kr[d];
          p[c] = acc * scale;
          if (p[c] > mx) mx = p[c];
        }
        double l = 0.0;
        for (int c = 0; c < cnt; ++c) {
          p[c] = exp(p[c] - mx);
          l += p[c];
        }
        for (int e = 0; e < dv; ++e) o[e] = 0.0;
        for (int c = 0; c < cnt; ++c) {
          p[c] /= l;
          const double* vr = v + (((int64_t)b * G + g) * Tkv + keys[c]) * dv;
          for (int e = 0; e < dv; ++e) o[e] += p[c] * vr[e];
        }
        double D = 0.0;
        for (int e = 0; e < dv; ++e) D += o[e] * dor[e];
        for (int c = 0; c < cnt; ++c) {
          const int64_t kv = ((int64_t)b * G + g) * Tkv + keys[c];
          const double* kr = k + kv * dk;
          const double* vr = v + kv * dv;
          double dp = 0.0;
          for (int e = 0; e < dv; ++e) dp += dor[e] * vr[e];
          const double ds = p[c] * (dp - D);
          for (int d = 0; d < dk; ++d) {
            dqr[d] += scale * ds * kr[d];
            dkk[kv * dk + d] += scale * ds * qr[d];
          }
          for (int e = 0; e < dv; ++e) dvv[kv * dv + e] += p[c] * dor[e];
        }
      }
    }
  free(keys);
  free(mark);
  free(p);
  free(o);
  return 0;
}

/* ------------------------------------------------------ Eq. 8 -> top-n --- */
/* Sum of e[0..n) in the order the GPU kernel uses: 64 lane partials, lane L summing
 * the elements 256 s + 4 L + u (s ascending, then u = 0..3) -- the four consecutive
 * elements of each 1 KB row piece it holds -- then a butterfly over lane distance
 * 32, 16, 8, 4, 2, 1. */
static float lane_order_sum(const float* e, int n) {
  float part[64];
  for (int L = 0; L < 64; ++L) {
    float acc = 0.0f;
    for (int s = 0; 256 * s < n; ++s)
      for (int u = 0; u < 4; ++u) {
        const int i = 256 * s + 4 * L + u;
        if (i < n) acc += e[i];
      }
    part[L] = acc;
  }
  for (int off = 32; off >= 1; off >>= 1) {
    float nxt[64];
    for (int L = 0; L < 64; ++L) nxt[L] = part[L] + part[L ^ off];
    memcpy(part, nxt, sizeof(part));
  }
  return part[0];
}

/* q [B,H,T,dk] fp32, kc [B,G,dk,NB] fp32, block_ends [NB].
 * out_idx [B,G,T,n] int64.  p_cmp [B,H,T,NB] and p_slc [B,H,T,nsel] optional.
 * tmap (optional): row r of q is query position tmap[r].
 * Returns 0, or 1 on bad arguments. */
int oracle_score_topn(int B, int H, int G, int T, int dk, int NB, const float* q, const float* kc,
                      const int32_t* block_ends, float scale, int l, int d, int lprime, int n, int include_fixed,
                      int n_fixed, const int32_t* tmap, int64_t* out_idx, float* p_cmp, float* p_slc) {
  if (G <= 0 || H % G || d <= 0 || l % d || lprime % d || n < 0) return 1;
  const int hpg = H / G;
  const int a = l / d, s = lprime / d;
  const int nsel = (NB + s - 1) / s;
  float* sv = (float*)malloc(sizeof(float) * (size_t)(NB > 0 ? NB : 1));
  float* ps = (float*)malloc(sizeof(float) * (size_t)(nsel > 0 ? nsel : 1));
  float* agg = (float*)malloc(sizeof(float) * (size_t)(nsel > 0 ? nsel : 1));
  unsigned char* vis = (unsigned char*)malloc((size_t)(NB > 0 ? NB : 1));
  unsigned char* taken = (unsigned char*)malloc((size_t)(nsel > 0 ? nsel : 1));
  int64_t* cand = (int64_t*)malloc(sizeof(int64_t) * (size_t)(n + 4));
  if (!sv || !ps || !agg || !vis || !taken || !cand) return 1;
  for (int b = 0; b < B; ++b)
    for (int g = 0; g < G; ++g)
      for (int tr = 0; tr < T; ++tr) {
        const int t = tmap ? tmap[tr] : tr;
        int any = 0;
        for (int i = 0; i < NB; ++i) {
          vis[i] = block_ends[i] <= t;
          any |= vis[i];
        }
        if (!any && NB > 0) vis[0] = 1;
        for (int j = 0; j < nsel; ++j) agg[j] = 0.0f;
        for (int hh = 0; hh < hpg; ++hh) {
          const int h = g * hpg + hh;
          const float* qr = q + (((int64_t)b * H + h) * T + tr) * dk;
          const float* kg = kc + ((int64_t)b * G + g) * dk * NB;
          /* logits: sequential fused multiply-add over the feature axis */
          float mx = -INFINITY;
          for (int i = 0; i < NB; ++i) {
            if (!vis[i]) continue;
            float acc = 0.0f;
            for (int e = 0; e < dk; ++e) acc = fmaf(qr[e], kg[(int64_t)e * NB + i], acc);
            sv[i] = acc * scale;
            if (sv[i] > mx) mx = sv[i];
          }
          for (int i = 0; i < NB; ++i) sv[i] = vis[i] ? oracle_exp32(sv[i] - mx) : 0.0f;
          const float sum = lane_order_sum(sv, NB);
          /* normalised with the correctly rounded reciprocal of the sum (one multiply
           * per block) */
          const float rs = 1.0f / sum;
          for (int i = 0; i < NB; ++i) sv[i] = sv[i] * rs;
          if (p_cmp) memcpy(p_cmp + (((int64_t)b * H + h) * T + tr) * NB, sv, sizeof(float) * (size_t)NB);
          /* Eq. 9, accumulated in the reference's (m, n) order */
          for (int j = 0; j < nsel; ++j) {
            float acc = 0.0f;
            for (int m = 0; m < s; ++m)
              for (int nn = 0; nn < a; ++nn) {
                const int ci = s * j + m + nn;
                if (ci < NB) acc += sv[ci];
              }
            ps[j] = acc;
          }
          if (p_slc) memcpy(p_slc + (((int64_t)b * H + h) * T + tr) * nsel, ps, sizeof(float) * (size_t)nsel);
          /* Eq. 10: heads summed in head order */
          for (int j = 0; j < nsel; ++j) agg[j] += ps[j];
        }
        /* top-k by (score desc, index asc) == stable descending sort */
        const int kk = n < nsel ? n : nsel;
        memset(taken, 0, (size_t)nsel);
        int nc = 0;
        if (include_fixed && n_fixed > 0) {
          int64_t c1 = (t - lprime) >= 0 ? (t - lprime) / lprime : 0;
          cand[nc++] = 0;
          cand[nc++] = c1;
          cand[nc++] = t / lprime;
        }
        int64_t* out = out_idx + (((int64_t)b * G + g) * T + tr) * n;
        int64_t top[4096];
        for (int r = 0; r < kk && r < 4096; ++r) {
          int best = -1;
          for (int j = 0; j < nsel; ++j) {
            if (taken[j]) continue;
            if (best < 0 || agg[j] > agg[best]) best = j;
          }
          taken[best] = 1;
          top[r] = best;
        }
        int no = 0;
        /* fixed blocks first (de-duplicated), then the top-k in order */
        for (int c = 0; c < nc + kk && no < n; ++c) {
          const int64_t v = c < nc ? cand[c] : top[c - nc];
          int dup = 0;
          for (int u = 0; u < no; ++u) dup |= out[u] == v;
          if (!dup) out[no++] = v;
        }
        for (; no < n; ++no) out[no] = -1;
      }
  free(sv);
  free(ps);
  free(agg);
  free(vis);
  free(taken);
  free(cand);
  return 0;
}
