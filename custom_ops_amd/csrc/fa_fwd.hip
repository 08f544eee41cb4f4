// fa_fwd.hip — masked FlashAttention-2 forward for MI355X (gfx950 / CDNA4).
//
// O = softmax(Q·Kᵀ·scale + mask)·V, additive mask broadcast over heads, GQA.
// Semantics follow the reference op (Defyli/custom_ops):
//   - mask added to the scaled score, col >= Sk always blocked
//       csrc/fa/sm89/fa_fwd_kernel.h:284-310
//   - online softmax with the -inf guards (max == -inf → use 0; l == 0 → output 0)
//       csrc/fa/common/softmax.h:65-151
//   - P rounded to the input dtype before the PV product   fa_fwd_kernel.h:384
//   - split-KV: partial O normalised by the local l, LSE per row; empty split
//     → O = 0, LSE = -inf; combine weights exp(lse_s - max) / Σ
//       fa_fwd_kernel.h:483-494, 827-835, 1406-1545
//   - kv_head = h / (H / Hk)                               fa_fwd_kernel.h:114
//
// Design (MI355X-native, not a translation of the CuTe kernels):
//   * One workgroup = 4 wave64 = one tile of BM=128 query rows; each wave owns
//     32 query rows. KV tiles of BN=64 keys.
//   * The score tile is computed transposed, Sᵀ = K·Qᵀ, with
//     v_mfma_f32_32x32x16_{bf16,f16}: A = K rows from LDS, B = Q held in VGPRs
//     for the whole loop. In the 32x32 C layout a lane then owns ONE query row
//     (column lane%32) and 16 keys, so row max / row sum are in-lane plus one
//     exchange with lane^32.
//   * Oᵀ = Vᵀ·Pᵀ: the Sᵀ accumulators, rounded to bf16/fp16, are directly the
//     B operand of the PV MFMA (no LDS round trip for P). The A operand Vᵀ is
//     produced by transposing V in registers while staging it into LDS, with
//     the key order inside each 16-key group permuted so that every MFMA
//     operand read is one ds_read_b128.
//   * The mask tile is staged through LDS with coalesced 16-byte loads and a
//     permuted key order that makes each lane's 16 mask values contiguous.
//   * K/V/mask for tile n+1 are loaded into registers while tile n computes
//     (one LDS buffer, two barriers per tile, 2 workgroups per CU).
//   * Sk tails are predicated in-kernel (no padded copies); unaligned mask rows
//     (mask row stride % 8 != 0) use element loads.
//   * Linear workgroup ids are remapped so that consecutive logical tiles
//     (the m-blocks of one head, the heads of one GQA group) land on the same
//     XCD and share its L2.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "mi355_fa.h"

namespace mi355fa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = 128;      // query rows per workgroup
constexpr int kBN = 64;       // keys per KV tile
constexpr int kWaves = 4;     // wave64s per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kMaxSplits = 64;
constexpr float kLog2e = 1.4426950408889634f;

// ── element traits ───────────────────────────────────────────────────────────
template <bool BF16> struct Elt;
template <> struct Elt<true> {
  typedef bf16x8 v8;
  static __device__ __forceinline__ f32x16 mfma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Elt<false> {
  typedef f16x8 v8;
  static __device__ __forceinline__ f32x16 mfma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <typename To, typename From>
__device__ __forceinline__ To bitcast(const From& x) {
  static_assert(sizeof(To) == sizeof(From), "size mismatch");
  return __builtin_bit_cast(To, x);
}

// ── kernel parameters (device copy, passed by value) ──────────────────────────
struct KParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* mask;
  uint16_t* o;
  float* o_part;   // [splits][B*H][Sq][D] fp32 (split path)
  float* lse_part; // [splits][B*H][Sq]    fp32, log2 domain

  int64_t q_bs, q_hs, q_rs;
  int64_t k_bs, k_hs, k_rs;
  int64_t v_bs, v_hs, v_rs;
  int64_t o_bs, o_hs, o_rs;
  int64_t m_bs, m_rs;

  int b, h, ratio;   // ratio = H / Hk
  int sq, sk;
  int num_m;         // ceil(Sq / kBM)
  int num_n;         // ceil(Sk / kBN)
  int num_splits;
  int n_per_split;   // tiles per split
  int total;         // grid size (workgroups)
  int mask_vec;      // 1: mask rows 16-byte aligned → vector loads
  float scale_log2;  // scale * log2(e)
};

// Workgroup-id remap: the hardware hands linear id L to XCD (L % 8). Give each
// XCD a contiguous chunk of logical tile ids so neighbouring tiles share an L2.
__device__ __forceinline__ int xcd_remap(int L, int total) {
  constexpr int kXcd = 8;
  const int q = total / kXcd, r = total % kXcd;
  const int xcd = L % kXcd, local = L / kXcd;
  return (xcd < r) ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

// ── LDS layout ────────────────────────────────────────────────────────────────
//  sK  [kBN][D + 8]      K rows, 16-byte pad per row (bank spread for b128 reads)
//  sVt [D][kBN + 8]      Vᵀ; inside every 16-key group the key order is
//                        {0-3, 8-11, 4-7, 12-15} so lane-group g reads 8 keys at +8g
//  sM  [kBM][kBN + 8]    mask; inside every 32-key block lane-group g's 16 keys
//                        {g*4 + (i/4)*8 + i%4} are stored contiguously at +16g
template <int D> struct Smem {
  static constexpr int kKStride = D + 8;
  static constexpr int kVStride = kBN + 8;
  static constexpr int kMStride = kBN + 8;
  static constexpr int kKElems = kBN * kKStride;
  static constexpr int kVElems = D * kVStride;
  static constexpr int kMElems = kBM * kMStride;
  static constexpr int kBytes = 2 * (kKElems + kVElems + kMElems);
};

// Registers holding one KV tile in flight (global → regs → LDS).
template <int D> struct TileRegs {
  static constexpr int kKChunks = kBN * D / 8 / kThreads;   // 16-byte chunks per thread
  static constexpr int kVItems = 16 * (D / 8);              // (key quad, d chunk) items
  static constexpr int kMChunks = kBM * kBN / 8 / kThreads;
  u32x4 k[kKChunks];
  u32x4 v[4];
  u32x4 m[kMChunks];
};

template <int D>
__device__ __forceinline__ void load_tile(const KParams& p, TileRegs<D>& r, int tid, int n,
                                          const uint16_t* kbase, const uint16_t* vbase,
                                          const uint16_t* mbase, int m0) {
  const int key0 = n * kBN;
  // K: row-major chunks, 16 bytes each.
  constexpr int kCPR = D / 8;  // chunks per row
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kKChunks; ++i) {
    const int ci = tid + i * kThreads;
    const int row = ci / kCPR, c = ci % kCPR;
    const int key = key0 + row;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (key < p.sk) val = *reinterpret_cast<const u32x4*>(kbase + (int64_t)key * p.k_rs + c * 8);
    r.k[i] = val;
  }
  // V: thread owns 4 consecutive keys × 8 d-values, transposed at store time.
  if (tid < TileRegs<D>::kVItems) {
    const int a = tid % 16, c = tid / 16;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int key = key0 + 4 * a + kk;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (key < p.sk) val = *reinterpret_cast<const u32x4*>(vbase + (int64_t)key * p.v_rs + c * 8);
      r.v[kk] = val;
    }
  }
  // Mask: 8 consecutive keys of one row per chunk.
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kMChunks; ++i) {
    const int ci = tid + i * kThreads;
    const int row = ci / 8, qd = ci % 8;
    const int m = m0 + row;
    const int key = key0 + qd * 8;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (m < p.sq) {
      const uint16_t* src = mbase + (int64_t)m * p.m_rs + key;
      if (p.mask_vec && key + 8 <= p.sk) {
        val = *reinterpret_cast<const u32x4*>(src);
      } else {
        uint16_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = (key + j < p.sk) ? src[j] : (uint16_t)0;
        val[0] = e[0] | ((uint32_t)e[1] << 16);
        val[1] = e[2] | ((uint32_t)e[3] << 16);
        val[2] = e[4] | ((uint32_t)e[5] << 16);
        val[3] = e[6] | ((uint32_t)e[7] << 16);
      }
    }
    r.m[i] = val;
  }
}

template <int D>
__device__ __forceinline__ void store_tile(const TileRegs<D>& r, int tid, uint16_t* sK,
                                           uint16_t* sVt, uint16_t* sM) {
  typedef Smem<D> S;
  constexpr int kCPR = D / 8;
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kKChunks; ++i) {
    const int ci = tid + i * kThreads;
    const int row = ci / kCPR, c = ci % kCPR;
    *reinterpret_cast<u32x4*>(sK + row * S::kKStride + c * 8) = r.k[i];
  }
  if (tid < TileRegs<D>::kVItems) {
    const int a = tid % 16, c = tid / 16;
    // position of key 4a inside the permuted 16-key group
    const int pos = (a / 4) * 16 + (a % 2) * 8 + ((a / 2) % 2) * 4;
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) {
      const int w = dd / 2;
      const bool hi = dd & 1;
      uint32_t x0 = r.v[0][w], x1 = r.v[1][w], x2 = r.v[2][w], x3 = r.v[3][w];
      u32x2 out;
      if (hi) {
        out[0] = (x0 >> 16) | (x1 & 0xffff0000u);
        out[1] = (x2 >> 16) | (x3 & 0xffff0000u);
      } else {
        out[0] = (x0 & 0xffffu) | (x1 << 16);
        out[1] = (x2 & 0xffffu) | (x3 << 16);
      }
      *reinterpret_cast<u32x2*>(sVt + (c * 8 + dd) * S::kVStride + pos) = out;
    }
  }
#pragma unroll
  for (int i = 0; i < TileRegs<D>::kMChunks; ++i) {
    const int ci = tid + i * kThreads;
    const int row = ci / 8, qd = ci % 8;
    const int kb = qd / 4, ib = (qd % 4) * 4;
    uint16_t* dst = sM + row * S::kMStride + kb * 32 + ib;
    *reinterpret_cast<u32x2*>(dst) = u32x2{r.m[i][0], r.m[i][1]};       // keys 8qd+0..3 → g=0
    *reinterpret_cast<u32x2*>(dst + 16) = u32x2{r.m[i][2], r.m[i][3]};  // keys 8qd+4..7 → g=1
  }
}

template <bool BF16>
__device__ __forceinline__ f32x16 mask_to_f32(u32x4 lo, u32x4 hi) {
  typedef typename Elt<BF16>::v8 V8;
  f32x8 a = __builtin_convertvector(bitcast<V8>(lo), f32x8);
  f32x8 b = __builtin_convertvector(bitcast<V8>(hi), f32x8);
  f32x16 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) { r[i] = a[i]; r[8 + i] = b[i]; }
  return r;
}

template <int D, bool BF16, bool SPLIT>
__global__ __launch_bounds__(kThreads, 2) void fa_fwd_kernel(const KParams p) {
  typedef typename Elt<BF16>::v8 V8;
  typedef Smem<D> S;
  constexpr int KD = D / 16;  // MFMA k-steps over the head dim
  constexpr int DB = D / 32;  // 32-wide d blocks of the output

  extern __shared__ __align__(16) uint16_t smem[];
  uint16_t* sK = smem;
  uint16_t* sVt = sK + S::kKElems;
  uint16_t* sM = sVt + S::kVElems;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;

  // logical tile id → (b, h, split, m_block)
  int t = xcd_remap(blockIdx.x, p.total);
  const int mb = t % p.num_m;  t /= p.num_m;
  const int split = t % p.num_splits;  t /= p.num_splits;
  const int h = t % p.h;
  const int b = t / p.h;
  const int hk = h / p.ratio;

  const int m0 = mb * kBM;
  const int n_begin = split * p.n_per_split;
  const int n_end = min(n_begin + p.n_per_split, p.num_n);

  const uint16_t* qbase = p.q + (int64_t)b * p.q_bs + (int64_t)h * p.q_hs;
  const uint16_t* kbase = p.k + (int64_t)b * p.k_bs + (int64_t)hk * p.k_hs;
  const uint16_t* vbase = p.v + (int64_t)b * p.v_bs + (int64_t)hk * p.v_hs;
  const uint16_t* mbase = p.mask + (int64_t)b * p.m_bs;

  // Q for this lane's row, as the B operand of Sᵀ = K·Qᵀ (kept for the whole loop).
  const int qrow = m0 + wave * 32 + l32;
  V8 qreg[KD];
#pragma unroll
  for (int kd = 0; kd < KD; ++kd) {
    u32x4 val = {0u, 0u, 0u, 0u};
    if (qrow < p.sq) val = *reinterpret_cast<const u32x4*>(qbase + (int64_t)qrow * p.q_rs + kd * 16 + g * 8);
    qreg[kd] = bitcast<V8>(val);
  }

  f32x16 oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) oacc[i] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;

  TileRegs<D> regs;
  if (n_begin < n_end) load_tile<D>(p, regs, tid, n_begin, kbase, vbase, mbase, m0);

  for (int n = n_begin; n < n_end; ++n) {
    __syncthreads();
    store_tile<D>(regs, tid, sK, sVt, sM);
    __syncthreads();
    if (n + 1 < n_end) load_tile<D>(p, regs, tid, n + 1, kbase, vbase, mbase, m0);

    // ── Sᵀ = K·Qᵀ : two 32-key blocks ─────────────────────────────────────
    f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const V8 a = bitcast<V8>(*reinterpret_cast<const u32x4*>(
            sK + (kb * 32 + l32) * S::kKStride + kd * 16 + g * 8));
        s[kb] = Elt<BF16>::mfma(a, qreg[kd], s[kb]);
      }
    }

    // ── mask add (log2 domain), tail predicate, online softmax ───────────
    const uint16_t* mrow = sM + (wave * 32 + l32) * S::kMStride + g * 16;
    const bool tail = (n + 1) * kBN > p.sk;
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(mrow + kb * 32);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(mrow + kb * 32 + 8);
      const f32x16 mk = mask_to_f32<BF16>(lo, hi);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float x = s[kb][i] * p.scale_log2 + mk[i] * kLog2e;
        if (tail) {
          const int key = n * kBN + kb * 32 + (i / 4) * 8 + g * 4 + (i % 4);
          x = (key < p.sk) ? x : -INFINITY;
        }
        s[kb][i] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;

    float lsum = 0.f;
    V8 pb[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f32x8 p0, p1;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float e0 = __builtin_amdgcn_exp2f(s[kb][i] - m_use);
        const float e1 = __builtin_amdgcn_exp2f(s[kb][8 + i] - m_use);
        lsum += e0 + e1;
        p0[i] = e0;
        p1[i] = e1;
      }
      pb[kb * 2 + 0] = __builtin_convertvector(p0, V8);
      pb[kb * 2 + 1] = __builtin_convertvector(p1, V8);
    }
    l_run = l_run * alpha + lsum;
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] *= alpha;

    // ── Oᵀ += Vᵀ·Pᵀ ─────────────────────────────────────────────────────
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const V8 a = bitcast<V8>(*reinterpret_cast<const u32x4*>(
            sVt + (db * 32 + l32) * S::kVStride + j * 16 + g * 8));
        oacc[db] = Elt<BF16>::mfma(a, pb[j], oacc[db]);
      }
    }
  }

  // ── epilogue ────────────────────────────────────────────────────────────
  const float l = l_run + __shfl_xor(l_run, 32);
  const float inv = (l == 0.f || l != l) ? 1.f : 1.f / l;
  if (qrow >= p.sq) return;

  if constexpr (!SPLIT) {
    uint16_t* orow = p.o + (int64_t)b * p.o_bs + (int64_t)h * p.o_hs + (int64_t)qrow * p.o_rs;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        f32x4 v4;
#pragma unroll
        for (int i = 0; i < 4; ++i) v4[i] = oacc[db][q4 * 4 + i] * inv;
        typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
        typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
        u32x2 packed;
        if constexpr (BF16) packed = bitcast<u32x2>(__builtin_convertvector(v4, bf16x4));
        else packed = bitcast<u32x2>(__builtin_convertvector(v4, f16x4));
        *reinterpret_cast<u32x2*>(orow + db * 32 + q4 * 8 + g * 4) = packed;
      }
    }
  } else {
    const int64_t bh = (int64_t)b * p.h + h;
    const int64_t slab = (int64_t)p.b * p.h * p.sq;   // rows per split
    const int64_t prow = (int64_t)split * slab + bh * p.sq + qrow;
    float* op = p.o_part + prow * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        f32x4 v4;
#pragma unroll
        for (int i = 0; i < 4; ++i) v4[i] = oacc[db][q4 * 4 + i] * inv;
        *reinterpret_cast<f32x4*>(op + db * 32 + q4 * 8 + g * 4) = v4;
      }
    }
    if (g == 0) {
      p.lse_part[prow] = (l == 0.f || l != l) ? -INFINITY : m_run + __builtin_amdgcn_logf(l);
    }
  }
}

// ── split-KV combine ────────────────────────────────────────────────────────
struct CParams {
  const float* o_part;
  const float* lse_part;
  uint16_t* o;
  int64_t o_bs, o_hs, o_rs;
  int b, h, sq, num_splits;
  int64_t rows;  // B*H*Sq
};

// One thread = 4 consecutive d-values of one row. Weights w_s = 2^(lse_s - max) / Σ.
template <int D, bool BF16>
__global__ __launch_bounds__(256) void fa_combine_kernel(const CParams p) {
  constexpr int kTPR = D / 4;              // threads per row
  constexpr int kRows = 256 / kTPR;        // rows per workgroup
  const int tid = threadIdx.x;
  const int64_t row = (int64_t)blockIdx.x * kRows + tid / kTPR;
  const int c4 = tid % kTPR;
  if (row >= p.rows) return;
  const int64_t slab = p.rows;
  float mx = -INFINITY;
  for (int s = 0; s < p.num_splits; ++s) mx = fmaxf(mx, p.lse_part[s * slab + row]);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  if (mx != -INFINITY) {
    for (int s = 0; s < p.num_splits; ++s) {
      const float w = __builtin_amdgcn_exp2f(p.lse_part[s * slab + row] - mx);
      if (w > 0.f) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(p.o_part + (s * slab + row) * D + c4 * 4);
        acc += w * v;
        wsum += w;
      }
    }
  }
  const float inv = (wsum > 0.f) ? 1.f / wsum : 0.f;
  acc *= inv;
  const int64_t bh = row / p.sq;
  const int m = (int)(row % p.sq);
  const int b = (int)(bh / p.h), h = (int)(bh % p.h);
  uint16_t* dst = p.o + (int64_t)b * p.o_bs + (int64_t)h * p.o_hs + (int64_t)m * p.o_rs + c4 * 4;
  typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
  typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
  if constexpr (BF16) *reinterpret_cast<u32x2*>(dst) = bitcast<u32x2>(__builtin_convertvector(acc, bf16x4));
  else *reinterpret_cast<u32x2*>(dst) = bitcast<u32x2>(__builtin_convertvector(acc, f16x4));
}

// ════════════════════════════════════════════════════════════════════════════
// host side
// ════════════════════════════════════════════════════════════════════════════

static void set_err(char* err, size_t errlen, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
static void set_err(char* err, size_t errlen, const char* fmt, ...) {
  if (!err || errlen == 0) return;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(err, errlen, fmt, ap);
  va_end(ap);
}

struct DeviceInfo {
  int cus = 256;
  bool gfx950 = false;
  bool queried = false;
};

static DeviceInfo g_dev[64];
static std::mutex g_dev_mu;

static DeviceInfo device_info() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return DeviceInfo{};
  }
  std::lock_guard<std::mutex> lk(g_dev_mu);
  DeviceInfo& d = g_dev[dev];
  if (!d.queried) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) d.cus = n;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) {
      d.gfx950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    }
    (void)hipGetLastError();
    d.queried = true;
  }
  return d;
}

static int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Cost model T(s) = ceil(nb/s)·K + s·P (structure of the reference's
// fa_mask_sm89_num_splits, csrc/fa/fa_fwd_launch.h:137-170): split only when
// the grid of row tiles under-fills the chip; K = relative cost of one KV tile
// in the main kernel, P = per-split cost of the partial write + combine.
static int cost_model_splits(int total_mblocks, int nb, int block_m, int d, int cus) {
  if (cus <= 0) cus = 1;
  if (total_mblocks <= 0 || nb <= 0) return 1;
  if (total_mblocks >= 0.8f * cus) return 1;
  if (nb <= 4) return 1;
  const float K = (d == 128) ? 2.25f : 2.5f;
  const int combine_units = total_mblocks * (block_m / 32) * (d / 32);
  const float P = fmaxf(0.35f, (float)combine_units / (float)cus);
  const float s_star = sqrtf((float)nb * K / P);
  const int cap_fill = (2 * cus) / total_mblocks > 1 ? (2 * cus) / total_mblocks : 1;
  int hi = (int)s_star + 8;
  if (hi > kMaxSplits) hi = kMaxSplits;
  if (hi > nb) hi = nb;
  if (hi > cap_fill) hi = cap_fill;
  int lo = (int)s_star - 8;
  if (lo < 1) lo = 1;
  if (lo > hi) lo = hi;
  int best = 1;
  float best_cost = 1e30f;
  for (int s = lo; s <= hi; ++s) {
    const float cost = (float)ceil_div(nb, s) * K + (float)s * P;
    if (cost < best_cost) { best_cost = cost; best = s; }
  }
  if (best < 1) best = 1;
  if (best > nb) best = nb;
  return best;
}

struct Plan {
  int num_m, num_n, splits, n_per_split;
  size_t o_part_bytes, lse_bytes, ws_bytes;
};

static Plan make_plan(const mi355_fa_params* p, int cus) {
  Plan pl{};
  pl.num_m = ceil_div(p->seqlen_q, kBM);
  pl.num_n = ceil_div(p->seqlen_k, kBN);
  int s = p->num_splits;
  if (s <= 0) {
    const char* env = getenv("MI355_FA_NUM_SPLITS");
    if (env && atoi(env) > 0) s = atoi(env);
  }
  if (s <= 0) s = cost_model_splits(p->b * p->h * pl.num_m, pl.num_n, kBM, p->d, cus);
  if (s > kMaxSplits) s = kMaxSplits;
  if (s > pl.num_n) s = pl.num_n;
  if (s < 1) s = 1;
  pl.splits = s;
  pl.n_per_split = (s > 1) ? ceil_div(pl.num_n, s) : pl.num_n;
  if (s > 1) {
    const size_t rows = (size_t)s * p->b * p->h * p->seqlen_q;
    pl.o_part_bytes = (rows * p->d * sizeof(float) + 255) & ~(size_t)255;
    pl.lse_bytes = (rows * sizeof(float) + 255) & ~(size_t)255;
    pl.ws_bytes = pl.o_part_bytes + pl.lse_bytes;
  }
  return pl;
}

static int validate(const mi355_fa_params* p, char* err, size_t errlen) {
  if (!p) { set_err(err, errlen, "params must not be NULL"); return MI355_FA_EINVAL; }
  if (p->dtype != MI355_FA_FP16 && p->dtype != MI355_FA_BF16) {
    set_err(err, errlen, "q must be float16 or bfloat16");
    return MI355_FA_EINVAL;
  }
  if (p->d != 64 && p->d != 128) {
    set_err(err, errlen, "Only head_dim=64 or head_dim=128 is supported");
    return MI355_FA_EINVAL;
  }
  if (p->b < 0 || p->h < 0 || p->h_k < 0 || p->seqlen_q < 0 || p->seqlen_k < 0) {
    set_err(err, errlen, "negative dimension");
    return MI355_FA_EINVAL;
  }
  if (p->h_k == 0 || p->h % p->h_k != 0) {
    set_err(err, errlen, "n_heads must be divisible by n_kv_heads (GQA)");
    return MI355_FA_EINVAL;
  }
  if (p->mask_seqlen_q < p->seqlen_q || p->mask_seqlen_k < p->seqlen_k) {
    set_err(err, errlen, "mask shape must be (B, 1, >=Sq, k-dim >= Sk)");
    return MI355_FA_EINVAL;
  }
  if (!(p->scale_softmax > 0.f) || isinf(p->scale_softmax)) {
    set_err(err, errlen, "scale_softmax must be a positive finite value");
    return MI355_FA_EINVAL;
  }
  const bool empty = (p->b == 0 || p->h == 0 || p->seqlen_q == 0);
  if (!empty) {
    if (!p->q || !p->o || (p->seqlen_k > 0 && (!p->k || !p->v || !p->mask))) {
      set_err(err, errlen, "tensor pointer is NULL");
      return MI355_FA_EINVAL;
    }
    // 16-byte vector access to q/k/v/o rows
    const uintptr_t al = (uintptr_t)p->q | (uintptr_t)p->o | (uintptr_t)p->k | (uintptr_t)p->v;
    const int64_t st = p->q_batch_stride | p->q_head_stride | p->q_row_stride | p->k_batch_stride |
                       p->k_head_stride | p->k_row_stride | p->v_batch_stride | p->v_head_stride |
                       p->v_row_stride;
    if ((al & 15) || (st & 7) || ((p->o_batch_stride | p->o_head_stride | p->o_row_stride) & 3)) {
      set_err(err, errlen, "q/k/v/o must be 16-byte aligned with strides that are multiples of 8 elements");
      return MI355_FA_EINVAL;
    }
    if ((uintptr_t)p->mask & 1) {
      set_err(err, errlen, "mask must be 2-byte aligned");
      return MI355_FA_EINVAL;
    }
  }
  return MI355_FA_OK;
}

template <int D, bool BF16>
static hipError_t launch(const KParams& kp, const CParams& cp, bool split, hipStream_t st) {
  const size_t smem = Smem<D>::kBytes;
  if (split) {
    hipLaunchKernelGGL((fa_fwd_kernel<D, BF16, true>), dim3(kp.total), dim3(kThreads), smem, st, kp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    constexpr int kRows = 256 / (D / 4);
    const int64_t blocks = (cp.rows + kRows - 1) / kRows;
    hipLaunchKernelGGL((fa_combine_kernel<D, BF16>), dim3((unsigned)blocks), dim3(256), 0, st, cp);
  } else {
    hipLaunchKernelGGL((fa_fwd_kernel<D, BF16, false>), dim3(kp.total), dim3(kThreads), smem, st, kp);
  }
  return hipGetLastError();
}

}  // namespace mi355fa

using namespace mi355fa;

extern "C" {

int mi355_fa_abi_version(void) { return MI355_FA_ABI_VERSION; }

const char* mi355_fa_build_info(void) {
  return "mi355_fa gfx950 BM=128 BN=64 waves=4 mfma32x32x16 splitkv+combine";
}

int mi355_fa_cost_model_splits(int total_mblocks, int num_n_blocks, int block_m, int head_dim,
                               int num_cus) {
  return cost_model_splits(total_mblocks, num_n_blocks, block_m, head_dim, num_cus);
}

int mi355_fa_num_splits(const mi355_fa_params* p) {
  if (!p || p->d <= 0) return 1;
  return make_plan(p, device_info().cus).splits;
}

size_t mi355_fa_workspace_bytes(const mi355_fa_params* p) {
  if (!p || p->d <= 0 || p->seqlen_q <= 0 || p->b <= 0 || p->h <= 0) return 0;
  return make_plan(p, device_info().cus).ws_bytes;
}

int mi355_fa_fwd(const mi355_fa_params* p, void* stream, char* err, size_t errlen) {
  int rc = validate(p, err, errlen);
  if (rc) return rc;
  if (p->b == 0 || p->h == 0 || p->seqlen_q == 0) return MI355_FA_OK;
  const DeviceInfo dev = device_info();
  if (!dev.gfx950) {
    set_err(err, errlen, "mi355_fa: current HIP device is not gfx950 (MI355X)");
    return MI355_FA_EDEVICE;
  }
  const Plan pl = make_plan(p, dev.cus);
  const int64_t total = (int64_t)p->b * p->h * pl.num_m * pl.splits;
  if (total >= (1LL << 24)) {
    set_err(err, errlen, "problem too large: %lld workgroups", (long long)total);
    return MI355_FA_EINVAL;
  }
  const bool split = pl.splits > 1;
  if (split && (!p->workspace || p->workspace_bytes < pl.ws_bytes)) {
    set_err(err, errlen, "split-KV needs %zu workspace bytes, got %zu", pl.ws_bytes, p->workspace_bytes);
    return MI355_FA_EWORKSPACE;
  }

  KParams kp{};
  kp.q = (const uint16_t*)p->q;
  kp.k = (const uint16_t*)p->k;
  kp.v = (const uint16_t*)p->v;
  kp.mask = (const uint16_t*)p->mask;
  kp.o = (uint16_t*)p->o;
  kp.q_bs = p->q_batch_stride; kp.q_hs = p->q_head_stride; kp.q_rs = p->q_row_stride;
  kp.k_bs = p->k_batch_stride; kp.k_hs = p->k_head_stride; kp.k_rs = p->k_row_stride;
  kp.v_bs = p->v_batch_stride; kp.v_hs = p->v_head_stride; kp.v_rs = p->v_row_stride;
  kp.o_bs = p->o_batch_stride; kp.o_hs = p->o_head_stride; kp.o_rs = p->o_row_stride;
  kp.m_bs = p->mask_batch_stride; kp.m_rs = p->mask_row_stride;
  kp.b = p->b; kp.h = p->h; kp.ratio = p->h / p->h_k;
  kp.sq = p->seqlen_q; kp.sk = p->seqlen_k;
  kp.num_m = pl.num_m; kp.num_n = pl.num_n;
  kp.num_splits = pl.splits; kp.n_per_split = pl.n_per_split;
  kp.total = (int)total;
  kp.mask_vec = (((uintptr_t)p->mask & 15) == 0 && (p->mask_batch_stride & 7) == 0 &&
                 (p->mask_row_stride & 7) == 0) ? 1 : 0;
  kp.scale_log2 = p->scale_softmax * kLog2e;

  CParams cp{};
  if (split) {
    kp.o_part = (float*)p->workspace;
    kp.lse_part = (float*)((char*)p->workspace + pl.o_part_bytes);
    cp.o_part = kp.o_part;
    cp.lse_part = kp.lse_part;
    cp.o = kp.o;
    cp.o_bs = kp.o_bs; cp.o_hs = kp.o_hs; cp.o_rs = kp.o_rs;
    cp.b = p->b; cp.h = p->h; cp.sq = p->seqlen_q; cp.num_splits = pl.splits;
    cp.rows = (int64_t)p->b * p->h * p->seqlen_q;
  }

  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  const bool bf16 = p->dtype == MI355_FA_BF16;
  if (p->d == 128) e = bf16 ? launch<128, true>(kp, cp, split, st) : launch<128, false>(kp, cp, split, st);
  else e = bf16 ? launch<64, true>(kp, cp, split, st) : launch<64, false>(kp, cp, split, st);
  if (e != hipSuccess) {
    set_err(err, errlen, "mi355_fa launch failed: %s", hipGetErrorString(e));
    return MI355_FA_ELAUNCH;
  }
  return MI355_FA_OK;
}

}  // extern "C"
