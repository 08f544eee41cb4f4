/*
 * fa_oracle.c — CPU restatement of the reference's masked FlashAttention-2
 * forward. TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg as the checker / CPU baseline, never by the
 * product path (custom_ops_amd/ must not load this library).
 *
 * What it restates (Defyli/custom_ops):
 *   - score x = q·k + mask·(1/scale), col >= Sk blocked
 *       csrc/fa/sm89/fa_fwd_kernel.h:284-310 (apply_mask_from_smem)
 *   - tile-wise online softmax in the unscaled domain:
 *       max_scaled = (max == -inf) ? 0 : max·scale_log2      csrc/fa/common/softmax.h:75
 *       p = exp2(x·scale_log2 − max_scaled)                   softmax.h:87
 *       rescale by exp2((m_prev − m_cur')·scale_log2), m_cur' = (m_cur == -inf ? 0 : m_cur)
 *                                                             softmax.h:118-126
 *       final inv = (sum == 0 || NaN) ? 1 : 1/sum; lse = m·scale + log(sum) or ∓inf
 *                                                             softmax.h:134-150
 *   - P rounded to the input dtype before P·V                 fa_fwd_kernel.h:384
 *   - split-KV partials (O normalised by the local l, rounded to the input
 *     dtype, empty split → O = 0 / LSE = -inf) and the LSE combine
 *       fa_fwd_kernel.h:495-524, 827-835, 1436-1470, 1472-1544
 *   - row-wise CPU structure and OpenMP over heads          csrc/fa/cpu/fa_fwd_cpu.cpp:78-224
 *   - Split-KV cost model                                     csrc/fa/fa_fwd_launch.h:137-170
 *
 * Inputs are fp32 arrays (callers widen bf16/fp16 exactly); the output is fp32.
 * p_round / o_round: 0 = keep fp32, 1 = round to bf16 (RNE), 2 = round to fp16 (RNE).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) return x; /* inf / nan */
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

/* IEEE binary16 round-to-nearest-even via the value grid (exact for |x| < 65520). */
static float round_fp16(float x) {
  if (x != x || isinf(x)) return x;
  float ax = fabsf(x);
  if (ax >= 65520.f) return x > 0 ? INFINITY : -INFINITY;
  int e;
  frexpf(ax, &e);              /* ax = f·2^e, f in [0.5,1) */
  int ulp_exp = e - 11;        /* 11 significant bits */
  if (ulp_exp < -24) ulp_exp = -24; /* subnormal spacing 2^-24 */
  float ulp = ldexpf(1.f, ulp_exp);
  float q = ax / ulp;
  float r = nearbyintf(q);     /* default rounding mode: nearest-even */
  float out = r * ulp;
  return x < 0 ? -out : out;
}

static float rnd(float x, int mode) {
  return mode == 1 ? round_bf16(x) : (mode == 2 ? round_fp16(x) : x);
}

float oracle_round(float x, int mode) { return rnd(x, mode); }

/* One query row over key range [n_lo, n_hi) in tiles of block_n, reference
 * online-softmax semantics. Writes o (normalised by local l) and the LSE
 * (natural-log domain, -inf when the row saw nothing), returns row_sum. */
static float row_range(const float* qr, const float* kh, const float* vh, const float* mr,
                       float* o, float* lse_out, int d, int sk_valid, int n_lo, int n_hi,
                       int block_n, float scale, int p_round, float* sbuf) {
  const float scale_log2 = scale * (float)M_LOG2E;
  const float inv_scale = 1.f / scale;
  float row_max = -INFINITY, row_sum = 0.f;
  int first = 1;
  for (int j = 0; j < d; ++j) o[j] = 0.f;
  for (int n0 = n_lo; n0 < n_hi; n0 += block_n) {
    const int n1 = (n0 + block_n < n_hi) ? n0 + block_n : n_hi;
    float tile_max = -INFINITY;
    for (int c = n0; c < n1; ++c) {
      float x;
      if (c >= sk_valid) {
        x = -INFINITY;
      } else {
        const float* kr = kh + (int64_t)c * d;
        float dot = 0.f;
        for (int j = 0; j < d; ++j) dot += qr[j] * kr[j];
        x = dot + mr[c] * inv_scale;
      }
      sbuf[c - n0] = x;
      if (x > tile_max) tile_max = x;
    }
    if (first) {
      row_max = tile_max;
      const float ms = (row_max == -INFINITY) ? 0.f : row_max * scale_log2;
      row_sum = 0.f;
      for (int c = n0; c < n1; ++c) {
        const float p = exp2f(sbuf[c - n0] * scale_log2 - ms);
        row_sum += p;
        sbuf[c - n0] = p;
      }
      first = 0;
    } else {
      const float prev = row_max;
      if (tile_max > row_max) row_max = tile_max;
      const float cur = (row_max == -INFINITY) ? 0.f : row_max;
      const float sc = exp2f((prev - cur) * scale_log2);
      row_sum *= sc;
      for (int j = 0; j < d; ++j) o[j] *= sc;
      const float ms = (row_max == -INFINITY) ? 0.f : row_max * scale_log2;
      for (int c = n0; c < n1; ++c) {
        const float p = exp2f(sbuf[c - n0] * scale_log2 - ms);
        row_sum += p;
        sbuf[c - n0] = p;
      }
    }
    for (int c = n0; c < n1; ++c) {
      const float p = rnd(sbuf[c - n0], p_round);
      if (p == 0.f) continue;
      const float* vr = vh + (int64_t)c * d;
      for (int j = 0; j < d; ++j) o[j] += p * vr[j];
    }
  }
  const int bad = (row_sum == 0.f || row_sum != row_sum);
  const float inv = bad ? 1.f : 1.f / row_sum;
  for (int j = 0; j < d; ++j) o[j] *= inv;
  if (lse_out) *lse_out = bad ? -INFINITY : row_max * scale + logf(row_sum);
  return row_sum;
}

/*
 * Full forward. q [B,H,Sq,d], k/v [B,Hk,Sk,d] dense; mask indexed as
 * mask[b*mask_bs + m*mask_rs + c] for c < Sk. num_splits <= 1: the base
 * kernel path; > 1: split-KV over ceil(nb/s)-tile ranges + LSE combine.
 * Output out [B,H,Sq,d] fp32 (not rounded to the dtype).
 */
void oracle_mha_fwd(const float* q, const float* k, const float* v, const float* mask,
                    float* out, int B, int H, int Hk, int Sq, int Sk, int d,
                    int64_t mask_bs, int64_t mask_rs, float scale, int p_round,
                    int block_n, int num_splits, int o_round) {
  const int ratio = H / Hk;
  const int nb = (Sk + block_n - 1) / block_n;
  if (num_splits < 1) num_splits = 1;
  const int n_per = (num_splits > 1) ? (nb + num_splits - 1) / num_splits : nb;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < H; ++h) {
      const int hk = h / ratio;
      const float* kh = k + ((int64_t)b * Hk + hk) * Sk * d;
      const float* vh = v + ((int64_t)b * Hk + hk) * Sk * d;
      float* sbuf = (float*)malloc(sizeof(float) * (block_n > 0 ? block_n : 1));
      float* part = (float*)malloc(sizeof(float) * (size_t)d * num_splits);
      float* lse = (float*)malloc(sizeof(float) * num_splits);
      for (int m = 0; m < Sq; ++m) {
        const float* qr = q + (((int64_t)b * H + h) * Sq + m) * d;
        const float* mr = mask + (int64_t)b * mask_bs + (int64_t)m * mask_rs;
        float* orow = out + (((int64_t)b * H + h) * Sq + m) * d;
        if (num_splits <= 1) {
          row_range(qr, kh, vh, mr, orow, NULL, d, Sk, 0, nb * block_n, block_n, scale, p_round,
                    sbuf);
          continue;
        }
        for (int s = 0; s < num_splits; ++s) {
          const int t0 = s * n_per;
          const int t1 = (t0 + n_per < nb) ? t0 + n_per : nb;
          float* po = part + (size_t)s * d;
          if (t0 >= t1) {
            for (int j = 0; j < d; ++j) po[j] = 0.f;
            lse[s] = -INFINITY;
            continue;
          }
          row_range(qr, kh, vh, mr, po, &lse[s], d, Sk, t0 * block_n, t1 * block_n, block_n,
                    scale, p_round, sbuf);
          for (int j = 0; j < d; ++j) po[j] = rnd(po[j], o_round);
        }
        float lmax = -INFINITY;
        for (int s = 0; s < num_splits; ++s) lmax = lse[s] > lmax ? lse[s] : lmax;
        const float lmax_c = (lmax == -INFINITY) ? 0.f : lmax;
        float sum = 0.f;
        for (int s = 0; s < num_splits; ++s) sum += expf(lse[s] - lmax_c);
        const float inv = (sum == 0.f || sum != sum) ? 0.f : 1.f / sum;
        for (int j = 0; j < d; ++j) orow[j] = 0.f;
        for (int s = 0; s < num_splits; ++s) {
          const float sc = expf(lse[s] - lmax_c) * inv;
          if (sc > 0.f)
            for (int j = 0; j < d; ++j) orow[j] += sc * part[(size_t)s * d + j];
        }
      }
      free(sbuf);
      free(part);
      free(lse);
    }
  }
}

/* Reference Split-KV cost model, csrc/fa/fa_fwd_launch.h:137-170, with the
 * per-architecture constants passed in (K for the kernel tile, P0 floor). */
int oracle_num_splits(int total_mblocks, int num_n_blocks, int block_m, int head_dim,
                      int num_sms, float K, float P0, int max_splits) {
  if (total_mblocks >= 0.8f * num_sms) return 1;
  if (num_n_blocks <= 4) return 1;
  const int combine = total_mblocks * (block_m / 32) * (head_dim / 32);
  float P = (float)combine / (float)num_sms;
  if (P < P0) P = P0;
  const float s_star = sqrtf((float)num_n_blocks * K / P);
  int cap_fill = (2 * num_sms) / (total_mblocks > 1 ? total_mblocks : 1);
  if (cap_fill < 1) cap_fill = 1;
  int hi = (int)s_star + 8;
  if (hi > max_splits) hi = max_splits;
  if (hi > num_n_blocks) hi = num_n_blocks;
  if (hi > cap_fill) hi = cap_fill;
  int lo = (int)s_star - 8;
  if (lo < 1) lo = 1;
  if (lo > hi) lo = hi;
  int best = 1;
  float best_cost = 1e30f;
  for (int s = lo; s <= hi; ++s) {
    const float cost = (float)((num_n_blocks + s - 1) / s) * K + (float)s * P;
    if (cost < best_cost) {
      best_cost = cost;
      best = s;
    }
  }
  if (best > num_n_blocks) best = num_n_blocks;
  return best < 1 ? 1 : best;
}
