// fa_fwd.hip — masked FlashAttention-2 forward for MI355X (gfx950 / CDNA4).
//
// O = softmax(Q·Kᵀ·scale + mask)·V, additive mask broadcast over heads, GQA.
// Semantics follow the reference op (Defyli/custom_ops):
//   - mask·(1/scale) added to the unscaled score q·k, col >= Sk always blocked
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
//   * One workgroup = WAVES wave64 (8 → BM = 256 query rows for grids that fill
//     the chip, 4 → BM = 128 for small grids and split-KV); each wave owns 32
//     query rows. KV tiles of BN = 64 keys.
//   * The score tile is computed transposed, Sᵀ = K·Qᵀ, with
//     v_mfma_f32_32x32x16_{bf16,f16}: A = K rows from LDS, B = Q held in VGPRs
//     for the whole loop. In the 32x32 C layout a lane then owns ONE query row
//     (column lane%32) and 16 keys, so row max / row sum are in-lane plus one
//     exchange with lane^32 (v_permlane32_swap).
//   * Oᵀ = Vᵀ·Pᵀ: the Sᵀ accumulators, rounded to bf16/fp16, are directly the
//     B operand of the PV MFMA (no LDS round trip for P). The A operand Vᵀ is
//     read from row-major V in LDS with ds_read_b64_tr_b16.
//   * The widened, pre-scaled mask tile initialises the QK accumulators, so no
//     pass over the scores sits between the two GEMMs except the row max.
//   * K, V and the mask tile of tile n+1 go HBM → LDS by buffer_load ... lds
//     (no VGPR staging, issued as inline assembly with explicit waits) while
//     tile n computes; two K/V stages, one barrier per tile. Each wave loads
//     its own 32 mask rows into a single buffer and widens the next tile's mask
//     before the barrier. XOR swizzles keep every LDS read conflict-free.
//   * Two waves per SIMD: one 8-wave workgroup, or two 4-wave workgroups, per CU.
//   * Lazy rescaling: the running max moves only when a score exceeds it by
//     more than 8 (log2 units); O and l are rescaled on those tiles only.
//   * Sk tails are predicated in-kernel (buffer-resource bounds return 0 for
//     K/V rows past Sk, scores of those keys are forced to -inf); unaligned mask
//     rows (mask row stride % 8 != 0) are loaded through registers.
//   * Linear workgroup ids are remapped so that consecutive logical tiles land
//     on the same XCD and share its L2: the m-blocks of one head (K/V reuse),
//     or for grids with few m-blocks the heads of one batch (mask reuse).

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <mutex>
#include <random>
#include <type_traits>

#include "mi355_fa.h"
#include "bits.h"

namespace mi355fa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBN = 64;          // keys per KV tile
constexpr int kMaxSplits = 64;
constexpr int kFuseMaxSplits = 2;   // the fused split tail serves launches of at most this many splits
constexpr int kCpolSc1 = 16;        // buffer cache policy: SC1 (device scope)
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

// ── buffer resources ──────────────────────────────────────────────────────────
// Raw buffer loads/stores with 32-bit offsets: the hardware returns 0 for reads
// (and drops writes) at offsets >= num_records. Each resource is bounded to the
// valid rows of one head / one batch, so K/V rows >= Sk, Q/O rows >= Sq and mask
// rows >= mask_seqlen_q need no predicate. All variable per-lane offsets are
// passed as the VGPR offset, which is what the range check covers; the per-tile
// shift along the keys moves the resource base instead (scalar arithmetic),
// shrinking num_records by the same amount so the check is unchanged.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void lds_void;
constexpr int kRsrcFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcFlags);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
}
// 16 bytes per lane from the buffer straight into LDS: lane i of the wave lands
// at lds + 16·i (gfx950 LDS DMA), no VGPR staging. Issued as inline assembly so
// the compiler does not track the LDS write: it would otherwise wait for every
// DMA in flight (vmcnt(0)) before each LDS read and each workgroup barrier,
// which serialises a multi-stage pipeline. Completion is therefore the
// caller's job: wait_vmcnt for the issuing wave, then wg_barrier for the others.
typedef int i32x4 __attribute__((ext_vector_type(4)));
// The same buffer descriptor as make_rsrc, as four plain words for the asm.
__device__ __forceinline__ i32x4 make_rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  // Uniform by construction; readfirstlane makes the compiler keep it in SGPRs.
  return i32x4{(int)__builtin_amdgcn_readfirstlane((uint32_t)a),
               (int)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu),
               (int)__builtin_amdgcn_readfirstlane(bytes), kRsrcFlags};
}
// LDS byte address of a __shared__ array (folds to a constant after inlining).
__device__ __forceinline__ uint32_t lds_addr(const uint16_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)p;
}
// NT: the non-temporal hint, for data each workgroup reads exactly once in a
// launch (the replacement policy then keeps other lines; cold reads of such a
// stream run up to 10 % faster).
template <bool NT = false>
__device__ __forceinline__ void bload16_lds(i32x4 rs, uint32_t lds_byte, uint32_t voff) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_byte);
  if constexpr (NT)
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen nt lds"
        :
        : "s"(m0v), "v"(voff), "s"(rs)
        : "memory", "m0");
  else
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, 0 offen lds"
        :
        : "s"(m0v), "v"(voff), "s"(rs)
        : "memory", "m0");
}

// ── kernel parameters (device copy, passed by value) ──────────────────────────
struct KParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* mask;
  uint16_t* o;
  uint16_t* o_part; // [splits][B*H][Sq][D] input dtype (split path)
  float* lse_part; // [splits][B*H][Sq]    fp32, natural log

  int64_t q_bs, q_hs;
  int64_t k_bs, k_hs;
  int64_t v_bs, v_hs;
  int64_t o_bs, o_hs;
  int64_t m_bs;
  int q_rs, k_rs, v_rs, o_rs, m_rs;  // row strides (elements)

  int b, h, ratio;   // ratio = H / Hk
  int pack;          // q-heads per workgroup (they share one KV head), divides ratio
  int sq, sk;
  int msq;           // mask rows present
  int num_m;         // ceil(Sq / BM)
  int num_n;         // ceil(Sk / kBN)
  int num_splits;
  int n_per_split;   // tiles per split
  int total;         // grid size (workgroups)
  int mask_direct;   // mask rows 16-byte aligned: the mask tile can go by LDS DMA
  int head_major;    // tile order: 1 heads fastest, 2 heads then splits fastest, 0 m-blocks fastest
  float scale;       // softmax scale (1/sqrt(d) in the reference op)
  // scale·log2(e) and the rescale slack in score units, as float bits: kernel
  // arguments arrive in SGPRs, which the assembly loops take as scalar operands
  uint32_t c2_bits, slack_bits;
  // Fused split tail (split launches with fuse set): every split counts itself
  // in on its row block's ticket word (48-bit launch tag above a 16-bit
  // count), and the last one combines the block; no combine launch follows.
  unsigned long long* tickets;
  unsigned long long tag;   // this launch's tag, below 2^48, never 0
  int fuse;
  uint32_t part_bytes, lse_bytes;   // sizes of o_part and lse_part (fuse: both below 2^31)
  int live;   // narrow each workgroup's key range to its live tiles
  // bf16, scale < 0.99: the compiled kernel's LDS mask path adds the mask on
  // the matrix core (bf16(1/scale) > 1.0078 makes -max_bf16 overflow to -inf)
  int mask_mfma;
  // K/V tiles are read by exactly one workgroup each: the compiled kernel
  // streams them with the non-temporal hint
  int kv_nt;
  // Live-tile map written by mask_stage_kernel before this launch (or null):
  // bit t % 8 of byte (b·map_slices + r / 16)·map_row_bytes + t / 8 is set
  // when tile t holds a visible entry of row r (rows in slices of 16). With it
  // the workgroups read their live ranges instead of scanning the mask.
  const uint8_t* live_map;
  int map_row_bytes;         // bytes per slice: ceil(num_n / 8)
  int map_slices;            // slices per batch: ceil(Sq / 16)
  // map_full_off bytes after the map: a byte per (batch, slice), 1 when tile 0
  // and the last tile both hold a visible entry of the slice's rows (the row
  // block's range is then the whole axis; its map bytes may be unwritten)
  int64_t map_full_off;
  uint8_t* live_map_out;     // the same map, for mask_stage_kernel
  // The mask as the caller passed it, for mask_stage_kernel: with a staged
  // copy, mask / m_bs / m_rs / msq above describe the copy instead
  const uint16_t* msrc;
  int64_t msrc_bs;
  int msrc_rs, msrc_q;
  uint16_t* stage_out;       // the staged copy [B][Sq][stage_rs] (or null)
  int stage_rs;              // ceil(Sk / 8) · 8
};

// Workgroup-id remap: the hardware hands linear id L to XCD (L % 8). Give each
// XCD a contiguous chunk of logical tile ids so neighbouring tiles share an L2.
__device__ __forceinline__ int xcd_remap(int L, int total) {
  constexpr int kXcd = 8;
  const int q = total / kXcd, r = total % kXcd;
  const int xcd = L % kXcd, local = L / kXcd;
  return (xcd < r) ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

// ── design ───────────────────────────────────────────────────────────────────
// Each wave owns 32 query rows and computes Sᵀ = K·Qᵀ with 32x32x16 MFMAs, so a
// lane holds the scores of ONE query row (its C column) and the row max / sum
// need only the lane 32 apart. Q stays in registers for the whole key loop.
//
// K rows are permuted in LDS: row r of a 32-key block holds key
// π(r) = ((r/4)%2)·16 + (r/8)·4 + r%4, so in the 32x32 C layout lane (query q,
// half g) owns the 16 CONSECUTIVE keys g·16 .. g·16+15 of the block. Mask
// reads, tail predicates and the PV operand order all follow from that: the
// exponentials of 8 consecutive keys form one bf16x8 B operand of Oᵀ += Vᵀ·Pᵀ.
__device__ __forceinline__ int key_perm(int r) {   // π within a 32-key block
  return ((r >> 2) & 1) * 16 + (r >> 3) * 4 + (r & 3);
}

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding: vmcnt[3:0] | [15:14])
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);   // no LDS access moves above the wait
}

// Workgroup barrier for the LDS pipeline: this wave's LDS reads have returned
// (so no other wave's DMA can overwrite what they read) and nothing moves across.
// Unlike __syncthreads it does not wait for the LDS DMAs in flight.
__device__ __forceinline__ void wg_barrier() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
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

// max / sum with the lane 32 apart (the other half of the same query row)
__device__ __forceinline__ float xhalf_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Σ of the 8 rounded P values of one MFMA operand, two per dot2 (fp32 accumulate).
template <bool BF16>
__device__ __forceinline__ float psum8(typename Elt<BF16>::v8 v, float acc) {
  if constexpr (BF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[2 * i], v[2 * i + 1]}, one, acc, false);
  } else {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_fdot2(f16x2{v[2 * i], v[2 * i + 1]}, one, acc, false);
  }
  return acc;
}

// Lazy rescaling: the running max used for the exponent only moves when a new
// score exceeds it by more than kRescaleSlack (natural-log units, = 8 in log2),
// so P stays <= 2^8 and the O/l rescale is skipped on almost every tile. The
// result is the same softmax: O and l are always scaled by the same factor.
constexpr float kRescaleSlack = 5.5451774f;   // 8·ln 2

// readfirstlane of a value the caller knows to be uniform
__device__ __forceinline__ int uni(int x) { return (int)__builtin_amdgcn_readfirstlane((uint32_t)x); }

struct TileIdx {
  int b, h, hk, split, m0, nb, ne;
};

// A workgroup of BM query rows serves p.pack heads that share one KV head
// (GQA), BM / p.pack rows of each: its K/V tiles serve every wave as before,
// and the waves of different heads read the same mask rows at the same time.
// tile_index gives the group's first head; place_wave moves one wave to its
// head h + w % pack and row slot w / pack.
template <int BM, class PT>
__device__ __forceinline__ TileIdx tile_index(PT& p) {
  TileIdx ti;
  int t = xcd_remap(blockIdx.x, p.total);
  const int ng = p.h / p.pack;   // head groups per batch
  int mb, hg;
  if (p.head_major == 2) {   // (b, m-block, split, head group): every workgroup reading a row block's mask runs together
    hg = t % ng;  t /= ng;
    ti.split = t % p.num_splits;  t /= p.num_splits;
    mb = t % p.num_m;
    ti.b = t / p.num_m;
  } else if (p.head_major) {   // (b, split, m-block, head group): the heads sharing a mask tile run together
    hg = t % ng;  t /= ng;
    mb = t % p.num_m;  t /= p.num_m;
    ti.split = t % p.num_splits;
    ti.b = t / p.num_splits;
  } else {              // (b, head group, split, m-block): the m-blocks sharing K/V run together
    mb = t % p.num_m;  t /= p.num_m;
    ti.split = t % p.num_splits;  t /= p.num_splits;
    hg = t % ng;
    ti.b = t / ng;
  }
  ti.h = hg * p.pack;
  ti.hk = ti.h / p.ratio;
  ti.m0 = mb * (BM / p.pack);
  ti.nb = ti.split * p.n_per_split;
  ti.ne = min(ti.nb + p.n_per_split, p.num_n);
  return ti;
}

// Wave w of a packed workgroup: head h + w % pack, rows from m0 + (w / pack)·rows.
// m0 is rebased so that m0 + w·rows stays the wave's first row (every row
// expression below is written that way; LDS slots stay indexed by w).
__device__ __forceinline__ void place_wave(TileIdx& ti, const KParams& p, int wave, int rows) {
  ti.h += wave % p.pack;
  ti.m0 += (wave / p.pack - wave) * rows;
}

// Live key range of a workgroup. A KV tile in which every mask entry of the
// workgroup's rows is -inf adds nothing to any of them (their scores there are
// all -inf: P = 0, and O, l and the running max are unchanged), so only the
// tiles from the first to the last one that holds a visible entry need to run,
// and the splits can share that range evenly instead of the whole key axis (an
// empty share runs no tile and leaves O = 0, LSE = -inf).
//  * live_probe: one 16-byte load per thread of the first and of the last tile
//    of the key axis (the first NT/8 rows of the workgroup), issued before the
//    kernel's own prologue loads so that one memory wait covers both.
//  * narrow_to_live: if the probe saw a visible entry at both ends (a dense
//    mask) the range is the whole axis and the nominal split ranges stand: the
//    cost is one OR over the workgroup. Otherwise the workgroup reads its rows'
//    mask from both ends, a window of U whole tiles per end and step (J
//    16-byte loads per thread and end per round, enough rounds to cover one
//    tile; once one end is found both windows serve the other), ORs the
//    per-tile verdicts over the workgroup and stops on each side at the first
//    tile with a visible entry: a sliding-window or causal mask reads its dead
//    edges once. Returns whether the range moved.
// Only entries that are exactly -inf count as blocked; columns >= Sk and rows
// >= Sq are ignored. A chunk read partly past the end of the buffer reads 0
// there, i.e. visible: that can only widen the range. Masks whose rows are not
// 16-byte aligned are read with the same (unaligned) 16-byte loads the
// compiled kernel's register mask path uses.
// U >= 1 (kRounds rounds cover a tile of BMAX >= rows rows), so every step
// either finds an end or moves it by at least one tile: the loop ends within
// num_n steps, uniformly over the workgroup (every wave reads the same words).
// Both functions read the parameters through the kernarg pointer passed
// through an empty asm statement: the compiler then cannot keep them in SGPRs
// across the tile loop (the assembly loops leave no registers to spill to).
// `red` is 4·waves words of LDS that no DMA touches until the final barrier
// (two sets, used alternately: a set is rewritten two steps after it was read,
// past the next barrier).
// Read that way (through a generic pointer) the fields count as divergent, so
// every field that forms a buffer descriptor or a branch goes through
// readfirstlane: a descriptor the compiler thinks divergent becomes a
// waterfall loop (one round trip per load), and a branch it thinks divergent
// makes every value defined under it divergent too.
typedef const KParams CKParams;
// A buffer descriptor whose words are uniform but were computed from values
// the compiler thinks divergent
__device__ __forceinline__ rsrc_t make_rsrc_uniform(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(low_u32(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(high_u32(a));
  return make_rsrc(reinterpret_cast<const void*>(compose_u64(lo, hi)),
                   __builtin_amdgcn_readfirstlane(bytes));
}
__device__ __forceinline__ CKParams& kernarg_params(const KParams& pk) {
#if defined(__HIP_DEVICE_COMPILE__)
  const KParams* kq = (const KParams*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(kq));
  return *kq;
#else
  return pk;   // host pass only: never runs
#endif
}

// whether the 8 entries of a chunk starting at column c0 hold a visible one
template <bool BF16>
__device__ __forceinline__ bool live8(u32x4 v, int c0, int sk) {
  // branch-free (a branch here lets the compiler sink a window load into it,
  // behind the step's wait: a second round trip per step)
  constexpr uint32_t kNeg = BF16 ? 0xff80u : 0xfc00u;
  const int nv = sk - c0;
  bool any = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    any |= (2 * i < nv) & ((v[i] & 0xffffu) != kNeg);
    any |= (2 * i + 1 < nv) & ((v[i] >> 16) != kNeg);
  }
  return any;
}

// OR over the wave: within each 16-lane row by DPP, over the four rows by
// readlane (a uniform result)
__device__ __forceinline__ uint32_t wave_or(uint32_t x) {
  x |= (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, false);    // quad_perm 1,0,3,2
  x |= (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, false);    // quad_perm 2,3,0,1
  x |= (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x124, 0xF, 0xF, false);   // row_ror 4
  x |= (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xF, 0xF, false);   // row_ror 8
  return __builtin_amdgcn_readlane(x, 0) | __builtin_amdgcn_readlane(x, 16) |
         __builtin_amdgcn_readlane(x, 32) | __builtin_amdgcn_readlane(x, 48);
}

// min and max over the wave, the same pattern as wave_or (a uniform result)
__device__ __forceinline__ int wave_min(int x) {
  x = min(x, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
  x = min(x, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
  x = min(x, __builtin_amdgcn_mov_dpp(x, 0x124, 0xF, 0xF, false));
  x = min(x, __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false));
  return min(min(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
             min(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}
__device__ __forceinline__ int wave_max(int x) {
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0x124, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false));
  return max(max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
             max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

// OR over the workgroup: wave_or, then one word per wave in LDS (set `set` of
// two), read by every thread after a barrier
template <int NT>
__device__ __forceinline__ void wg_or2(uint32_t& a, uint32_t& b, uint32_t* red, int set) {
  constexpr int kW = NT / 64;
  const uint32_t wa = wave_or(a), wb = wave_or(b);
  const int tid = threadIdx.x;
  uint32_t* w = red + 2 * kW * set;
  w[tid >> 6] = wa;
  w[kW + (tid >> 6)] = wb;
  __syncthreads();
  uint32_t ra = 0u, rb = 0u;
#pragma unroll
  for (int i = 0; i < kW; ++i) { ra |= w[i]; rb |= w[kW + i]; }
  a = __builtin_amdgcn_readfirstlane(ra);
  b = __builtin_amdgcn_readfirstlane(rb);
}

// The mask buffer of batch b
__device__ __forceinline__ rsrc_t mask_rsrc(CKParams& p, int b) {
  return make_rsrc_uniform(p.mask + (int64_t)b * p.m_bs, (uint32_t)p.msq * p.m_rs * 2u);
}

struct LiveProbe { u32x4 l, r; };

template <int NT, bool MAP = false, bool SCAN = true, bool LOCAL = false>
__device__ __forceinline__ LiveProbe live_probe(const TileIdx& ti, const KParams& pk) {
  CKParams& p = kernarg_params(pk);
  LiveProbe pr{};
  if (!SCAN || !uni(p.live)) return pr;
  if constexpr (MAP) {
    if (p.live_map) return pr;
  }
  const rsrc_t rm = mask_rsrc(p, ti.b);
  const int tid = threadIdx.x;
  const uint32_t rowoff = (uint32_t)(ti.m0 + (tid >> 3)) * (uint32_t)p.m_rs + (uint32_t)(tid & 7) * 8u;
  // LOCAL: the ends of the workgroup's own split range, else of the key axis
  const int t0 = LOCAL ? ti.nb : 0, t1 = LOCAL ? max(ti.ne - 1, 0) : p.num_n - 1;
  pr.l = bload16(rm, (rowoff + (uint32_t)t0 * kBN) * 2u);
  pr.r = bload16(rm, (rowoff + (uint32_t)t1 * kBN) * 2u);
  return pr;
}

// The live range of the workgroup's row block from the live-tile map: the
// first and the last set bit over the map slices of its rows (the same
// [lo, hi] the scan below finds, so the same split ranges and the same
// results).
template <int NT>
__device__ __forceinline__ bool range_from_map(TileIdx& ti, CKParams& p, int rows, uint32_t* red) {
  constexpr int kW = NT / 64;
  const int tid = threadIdx.x;
  const int nbytes = uni(p.map_row_bytes);
  const int s0 = ti.m0 >> 4, s1 = min((ti.m0 + rows + 15) >> 4, p.map_slices);
  const uint8_t* map = p.live_map + ((int64_t)ti.b * p.map_slices + s0) * nbytes;
  int mlo = 0x7fffffff, mhi = 0;
  for (int i = tid; i < (s1 - s0) * nbytes; i += NT) {
    const uint32_t v = map[i];
    if (v) {
      const int t0 = (i % nbytes) * 8;
      mlo = min(mlo, t0 + __builtin_ctz(v));
      mhi = max(mhi, t0 + 32 - __builtin_clz(v));   // one past the last
    }
  }
  // a slice flagged whole-axis: its bytes may be unwritten, the range is [0, num_n)
  const uint8_t* full = p.live_map + p.map_full_off + (int64_t)ti.b * p.map_slices + s0;
  for (int i = tid; i < s1 - s0; i += NT)
    if (full[i]) { mlo = 0; mhi = p.num_n; }
  // per wave by DPP, then one slot per wave (no LDS atomics: the compiler's
  // whole-wave reduction for them needs registers the assembly loops lack)
  mlo = wave_min(mlo);
  mhi = wave_max(mhi);
  int* w = reinterpret_cast<int*>(red);
  if ((tid & 63) == 0) {
    w[2 * (tid >> 6)] = mlo;
    w[2 * (tid >> 6) + 1] = mhi;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kW; ++i) {
    mlo = min(mlo, w[2 * i]);
    mhi = max(mhi, w[2 * i + 1]);
  }
  int lo = (int)__builtin_amdgcn_readfirstlane(mlo);
  int hi = min((int)__builtin_amdgcn_readfirstlane(mhi), p.num_n) - 1;
  __syncthreads();                         // every wave has read `red` before any DMA lands
  if (lo > hi) { lo = 0; hi = -1; }        // no visible entry in these rows
  if (lo == 0 && hi == p.num_n - 1) return false;   // whole axis live: the nominal ranges stand
  const int ns = uni(p.num_splits);
  const int per = (hi - lo + 1 + ns - 1) / ns;
  const int nb = min(lo + ti.split * per, hi + 1);
  ti.nb = nb;
  ti.ne = min(nb + per, hi + 1);
  return true;
}

// Pre-pass for a mask whose rows are not 16-byte aligned (a mask of
// Sk % 8 != 0 columns, or one that starts off a 16-byte boundary): one
// workgroup per (batch, 16 rows, 8 KV tiles) reads those rows' 512 columns
// once (rows < Sq, columns < Sk) and
//  * with stage_out, writes them to the staged copy [B][Sq][stage_rs], whose
//    rows are 16-byte aligned, the columns Sk .. stage_rs - 1 -inf: the
//    attention kernel then takes its mask tiles by LDS DMA, as from an
//    aligned mask (the reference pads the mask for Sk % 8 != 0 as well,
//    csrc/fa/fa_fwd_op.cu:117-134);
//  * with live_map_out, writes one map byte, bit t set when tile t of the
//    group has an entry that is not -inf: the launch's workgroups then read
//    their live ranges from the map (range_from_map) instead of each scanning
//    its rows' mask, which the 8 workgroups sharing an m-block on cfg5's shape
//    would each read again.
// Each wave takes one row's 512 columns per step and reads them as aligned
// 16-byte blocks from the 16-byte boundary at or below their start (lane i
// block i, lane 63 also block 64); lane i's 8 entries are the end of its
// block and the start of the next lane's (ds_bpermute), aligned by the row's
// byte offset, which is the same for the whole wave. Unaligned 16-byte loads
// ran at half the rate (8.4 MB: 6.5 against 3.7 µs for the map alone). The
// descriptor covers whole 16-byte blocks, from the block that holds the
// batch's first entry to the one that holds its last: those lie in the pages
// of the mask's own bytes, and no load reaches past the descriptor (a load
// that does reads 0 for its in-range bytes too, and 0 is visible). Entries of
// columns >= Sk and rows >= Sq are not counted; rows >= Sq are not staged, and
// the staged columns Sk .. stage_rs - 1 hold -inf. Every map byte and every
// staged chunk has one writer, so neither needs clearing.
template <bool BF16>
__global__ __launch_bounds__(256) void mask_stage_kernel(KParams p) {
  constexpr uint32_t kNegPair = BF16 ? 0xff80ff80u : 0xfc00fc00u;
  constexpr uint32_t kNeg = kNegPair & 0xffffu;
  constexpr int kThreads = 256, kRows = 16, kChunksPerRow = 8 * 8;   // 8 tiles x 8 chunks
  constexpr int kSteps = kRows * kChunksPerRow / kThreads;          // rows per wave
  const int g = blockIdx.x % p.map_row_bytes;          // 8-tile group
  const int sl = (blockIdx.x / p.map_row_bytes) % p.map_slices;
  const int b = blockIdx.x / (p.map_row_bytes * p.map_slices);
  const int r0 = sl * kRows;
  const int nr = min(kRows, p.sq - r0);
  const uintptr_t bsrc = reinterpret_cast<uintptr_t>(p.msrc + (int64_t)b * p.msrc_bs);
  const uintptr_t abase = bsrc & ~(uintptr_t)15;
  const uint32_t lead = (uint32_t)(bsrc - abase);
  const uint32_t nrec = (lead + (uint32_t)p.msrc_q * (uint32_t)p.msrc_rs * 2u + 15u) & ~15u;
  const rsrc_t rm = make_rsrc(reinterpret_cast<const void*>(abase), nrec);
  const int sk = p.sk;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint8_t* full_out = p.live_map_out ? p.live_map_out + p.map_full_off + (int64_t)b * p.map_slices + sl : nullptr;
  if (!p.stage_out) {
    // Map only: first a probe of the slice's rows in tile 0 (lanes k = 0-7 of
    // each 16) and in the last tile (k = 8-15; the chunk that holds Sk read
    // shifted back to end at column Sk - 1). Both live: the row block's range
    // is the whole axis, so the flag says so and the 8 tiles need no reading
    // (a dense mask reads 2 tiles per row). Every group's workgroup of the
    // slice computes the same flag.
    const int t = threadIdx.x, row = t >> 4, k = t & 15;
    const int c0 = (k < 8 ? 0 : (p.num_n - 1) * kBN) + 8 * (k & 7);
    const bool in = row < nr && c0 < sk;
    const int sh = max(c0 + 8 - sk, 0);
    const uint32_t off = lead + ((uint32_t)(r0 + row) * (uint32_t)p.msrc_rs + (uint32_t)(c0 - sh)) * 2u;
    const u32x4 pv = bload16(rm, in ? off : 0xfffffff0u);
    bool live = false;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      live |= (j >= sh) & (((pv[j >> 1] >> (16 * (j & 1))) & 0xffffu) != kNeg);
    live &= in;
    const bool l0 = __syncthreads_or(live && k < 8), l1 = __syncthreads_or(live && k >= 8);
    if (threadIdx.x == 0) *full_out = (l0 && l1) ? 1u : 0u;
    if (l0 && l1) return;
  } else if (full_out && threadIdx.x == 0) {
    *full_out = 0u;
  }
  u32x4 v[kSteps], x[kSteps];
  uint32_t dl[kSteps];
#pragma unroll
  for (int u = 0; u < kSteps; ++u) {
    const int row = u * (kThreads / 64) + wave;       // wave-uniform
    const uint32_t seg = lead + ((uint32_t)(r0 + row) * (uint32_t)p.msrc_rs + (uint32_t)(g * 8 * kBN)) * 2u;
    const uint32_t a = seg & ~15u;
    dl[u] = seg - a;                                  // 0 .. 14, even
    const bool in = row < nr;
    // outside: an out-of-range offset, which reads 0 without an access
    v[u] = bload16(rm, in ? a + 16u * (uint32_t)lane : 0xfffffff0u);
    x[u] = bload16(rm, (in && lane == 63) ? a + 1024u : 0xfffffff0u);
  }
  uint32_t mine = 0u;
#pragma unroll
  for (int u = 0; u < kSteps; ++u) {
    const int row = u * (kThreads / 64) + wave;
    const int c0 = g * 8 * kBN + 8 * lane;
    u32x4 nx;   // the next lane's block (lane 63: its own second load)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t t = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane + 1) & 63) * 4, (int)v[u][i]);
      nx[i] = lane == 63 ? x[u][i] : t;
    }
    const uint32_t cat[8] = {v[u][0], v[u][1], v[u][2], v[u][3], nx[0], nx[1], nx[2], nx[3]};
    const uint32_t q = dl[u] >> 2, sh = dl[u] & 3u;   // whole words, then bytes
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t lo = cat[j], hi = cat[j + 1];
#pragma unroll
      for (int k = 1; k < 4; ++k)
        if (q == (uint32_t)k) { lo = cat[j + k]; hi = cat[j + k + 1]; }
      w[j] = __builtin_amdgcn_alignbyte(hi, lo, sh);
    }
    if (row >= nr || c0 >= sk) continue;
    if (c0 + 8 > sk) {   // the chunk that holds Sk: -inf from column Sk on
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (c0 + j >= sk)
          w[j >> 1] = (j & 1) ? ((w[j >> 1] & 0xffffu) | (kNeg << 16)) : ((w[j >> 1] & 0xffff0000u) | kNeg);
    }
    const bool live = !((w[0] == kNegPair) & (w[1] == kNegPair) & (w[2] == kNegPair) & (w[3] == kNegPair));
    if (live) mine |= 1u << (lane >> 3);
    if (p.stage_out)
      *reinterpret_cast<u32x4*>(p.stage_out + ((int64_t)b * p.sq + r0 + row) * p.stage_rs + c0) = w;
  }
  if (!p.live_map_out) return;
  __shared__ uint32_t bits;
  if (threadIdx.x == 0) bits = 0u;
  __syncthreads();
  mine = wave_or(mine);   // one LDS atomic per wave, not per thread
  if ((threadIdx.x & 63) == 0 && mine) atomicOr(&bits, mine);
  __syncthreads();
  if (threadIdx.x == 0)
    p.live_map_out[((int64_t)b * p.map_slices + sl) * p.map_row_bytes + g] = (uint8_t)bits;
}

// range_from_map for the assembly loops: every wave reads its row block's map
// bytes itself and reduces them by DPP (no LDS, no barrier, few SGPRs).
__device__ __forceinline__ bool range_from_map_wave(TileIdx& ti, CKParams& p, int rows) {
  const int lane = threadIdx.x & 63;
  const int nbytes = p.map_row_bytes;
  const int s0 = ti.m0 >> 4, s1 = min((ti.m0 + rows + 15) >> 4, p.map_slices);
  const uint8_t* map = p.live_map + ((int64_t)ti.b * p.map_slices + s0) * nbytes;
  int mlo = 0x7fffffff, mhi = 0;
  for (int i = lane; i < (s1 - s0) * nbytes; i += 64) {
    const uint32_t v = map[i];
    if (v) {
      const int t0 = (i % nbytes) * 8;
      mlo = min(mlo, t0 + __builtin_ctz(v));
      mhi = max(mhi, t0 + 32 - __builtin_clz(v));   // one past the last
    }
  }
  // a slice flagged whole-axis: its bytes may be unwritten, the range is [0, num_n)
  const uint8_t* full = p.live_map + p.map_full_off + (int64_t)ti.b * p.map_slices + s0;
  for (int i = lane; i < s1 - s0; i += 64)
    if (full[i]) { mlo = 0; mhi = p.num_n; }
  int lo = wave_min(mlo), hi = min(wave_max(mhi), p.num_n) - 1;
  if (lo > hi) { lo = 0; hi = -1; }        // no visible entry in these rows
  if (lo == 0 && hi == p.num_n - 1) return false;   // whole axis live: the nominal ranges stand
  const int ns = p.num_splits;
  const int per = (hi - lo + 1 + ns - 1) / ns;
  const int nb = min(lo + ti.split * per, hi + 1);
  ti.nb = nb;
  ti.ne = min(nb + per, hi + 1);
  return true;
}

// LOCAL (the compiled kernel): a split launch without a map narrows each
// workgroup's own nominal range [nb, ne) to its live tiles and keeps the
// nominal partition, so a workgroup scans only its own share of the mask.
// Scanning the whole axis to re-partition the live range (the assembly
// loops) reads a sparse mask's dead part once per split and head: a top-left
// causal [1,16,16,128,32768] took 357 µs that way on 16 splits.
template <bool BF16, int NT, int BMAX, int J, bool REUSE, bool MAP = false, bool SCAN = true, bool LOCAL = false>
__device__ __forceinline__ bool narrow_to_live(TileIdx& ti, const KParams& pk, int rows, const LiveProbe& pr,
                                               uint32_t* red) {
  CKParams& p = kernarg_params(pk);
  if (!uni(p.live)) return false;
  const int nr = uni(min(rows, p.sq - ti.m0));
  if (nr <= 0) return false;
  const int tid = threadIdx.x;
  const int nn = p.num_n;   // the scan's control stays in VGPRs: no SGPRs to spare here
  if constexpr (MAP) {
    if (p.live_map) {
      if constexpr (REUSE) return range_from_map<NT>(ti, p, rows, red);
      else return range_from_map_wave(ti, p, rows);
    }
  }
  if constexpr (!SCAN) return false;
  // the scanned range: the workgroup's own (LOCAL) or the whole key axis
  const int first = LOCAL ? ti.nb : 0, last = LOCAL ? ti.ne - 1 : nn - 1;
  if (LOCAL && first > last) return false;   // an empty share stays empty
  // the probe's verdict: tile first / tile last live in the chunks it read
  uint32_t lb = ((tid < nr * 8) & live8<BF16>(pr.l, first * kBN + (tid & 7) * 8, p.sk)) ? 1u : 0u;
  uint32_t rb = ((tid < nr * 8) & live8<BF16>(pr.r, last * kBN + (tid & 7) * 8, p.sk)) ? 1u : 0u;
  wg_or2<NT>(lb, rb, red, 1);
  if (lb && rb) {                          // both ends live: the nominal ranges stand
    __syncthreads();                       // every wave has read `red` before any DMA lands
    return false;
  }
  int lo = lb ? first : -1, hi = rb ? last : -1;
  constexpr int kRounds = (8 * BMAX + J * NT - 1) / (J * NT);   // rounds that cover one whole tile
  constexpr int NL = kRounds * J;
  const int cpt = nr * 8;                  // 16-byte chunks per tile of these rows
  int U = (kRounds * J * NT) / cpt;        // tiles per window: 1 .. 32
  U = U > 32 ? 32 : U;
  const rsrc_t rm = mask_rsrc(p, ti.b);
  // Each thread's chunks, the same in every step: window slot t, row offset
  // and column within the tile (one division each, here, not per step)
  int tj[NL];
  uint32_t roff[NL];
#pragma unroll
  for (int n = 0; n < NL; ++n) {
    const int c = n * NT + tid, t = c / cpt, rem = c - t * cpt;
    tj[n] = t;
    roff[n] = (uint32_t)(ti.m0 + (rem >> 3)) * (uint32_t)p.m_rs + (uint32_t)(rem & 7) * 8u;
  }
  const int c0 = (tid & 7) * 8;   // NT and cpt are multiples of 8: rem & 7 == tid & 7
  const int sk = p.sk;
  int L = first, R = last;
  for (int step = 0; lo < 0 || hi < 0; ++step) {
    if (L > R) break;                      // every tile scanned and dead
    // Two windows of U tile slots. While both ends are open, slots A read
    // tiles L, L+1, .. and slots B tiles R, R-1, ..; once one end is found,
    // both windows serve the other end (2U tiles per step).
    const int rem_t = R - L + 1;
    const bool both = !REUSE || (lo < 0 && hi < 0), left = lo < 0;
    // REUSE off (the assembly loops, whose prologue has no SGPRs to spare):
    // window A serves the left end while it is open, B the right end
    const int ua = (REUSE || lo < 0) ? min(U, rem_t) : 0;
    const int ub = both ? ((REUSE || hi < 0) ? min(U, rem_t) : 0) : min(U, max(rem_t - U, 0));
    // tile of slot t in window A / B: base + dir·t
    const int da = (!REUSE || left) ? 1 : -1, a0 = (!REUSE || left) ? L : R;
    const int db = (both || !left) ? -1 : 1, b0 = both ? R : (left ? L + U : R - U);
    uint32_t abits = 0u, bbits = 0u;
    // branch-free: a chunk outside its window loads tile L (in range) and is
    // ignored
    u32x4 va[NL], vb[NL];
#pragma unroll
    for (int n = 0; n < NL; ++n) {
      const int t = tj[n];
      va[n] = bload16(rm, (roff[n] + (uint32_t)(t < ua ? a0 + da * t : L) * kBN) * 2u);
      vb[n] = bload16(rm, (roff[n] + (uint32_t)(t < ub ? b0 + db * t : L) * kBN) * 2u);
    }
#pragma unroll
    for (int n = 0; n < NL; ++n) {
      const int t = tj[n];
      const uint32_t bit = 1u << (t & 31);
      abits |= ((t < ua) & live8<BF16>(va[n], (a0 + da * t) * kBN + c0, sk)) ? bit : 0u;
      bbits |= ((t < ub) & live8<BF16>(vb[n], (b0 + db * t) * kBN + c0, sk)) ? bit : 0u;
    }
    wg_or2<NT>(abits, bbits, red, step & 1);
    if (both) {
      if (lo < 0) { if (abits) lo = L + __builtin_ctz(abits); else L += ua; }
      if (hi < 0) { if (bbits) hi = R - __builtin_ctz(bbits); else R -= ub; }
    } else if (left) {                     // A: tiles L .. L+ua-1, B: L+U .. L+U+ub-1
      if (abits) lo = L + __builtin_ctz(abits);
      else if (bbits) lo = L + U + __builtin_ctz(bbits);
      else L += ua + ub;
    } else {                               // A: tiles R .. R-ua+1, B: R-U .. R-U-ub+1
      if (abits) hi = R - __builtin_ctz(abits);
      else if (bbits) hi = R - U - __builtin_ctz(bbits);
      else R -= ua + ub;
    }
  }
  __syncthreads();                         // every wave has read `red` before any DMA lands
  if constexpr (LOCAL) {
    if (lo < 0) { lo = first; hi = first - 1; }   // no visible entry: an empty range
    ti.nb = lo;
    ti.ne = hi + 1;
    return true;
  }
  // no visible entry in these rows: an empty range (lo = 0, hi = -1)
  if (lo < 0) { lo = 0; hi = -1; }
  const int ns = uni(p.num_splits);
  const int per = (hi - lo + 1 + ns - 1) / ns;
  const int nb = min(lo + ti.split * per, hi + 1);
  ti.nb = nb;
  ti.ne = min(nb + per, hi + 1);
  return true;
}

// ── main kernel: 32 query rows per wave, WAVES = 4 or 8 waves ─────────────────
// A wave needs 210-245 registers (two waves per SIMD fit); with 8 waves
// (BM = 256) two waves share every SIMD, hiding each other's LDS and MFMA
// latencies. 4 waves (BM = 128) serve small grids and split-KV. K, V and the
// mask tile arrive by LDS DMA; V is read transposed.
//  sK   [kBN][D]    unit c of row r at slot c ^ (r % UPR)   (π-permuted rows)
//  sV   [kBN][D]    natural key order, unit c of row r at slot c ^ swzV(r); the
//                   PV operand Vᵀ is read with ds_read_b64_tr_b16 (in each 16-lane
//                   group, source lane s reads 4 d-values of key base + s/4 and
//                   output lane o receives keys base..base+3 of column D0 + o)
template <int D, int WAVES> struct Geo {
  static constexpr int kWaves = WAVES;
  static constexpr int kBM = 32 * WAVES;
  static constexpr int kThreads = 64 * WAVES;
  static constexpr int kUPR = D / 8;
  static constexpr int kKElems = kBN * D;
  static constexpr int kVElems = kBN * D;
  static constexpr int kMElems = kBM * kBN;
  static constexpr int kMWaveLoads = kBM * 8 / 64 / kWaves;
  static constexpr int kKWaveLoads = kBN * kUPR / 64 / kWaves;
};

template <int D> __device__ __forceinline__ int v_swz(int r) {
  return (D == 128) ? 4 * (r & 3) : 4 * ((r >> 1) & 1);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int mask_swz(int m) { return (m >> 1) & 7; }
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// O (or a split's partial O) of 32 query rows, normalised by l and rounded to
// the input dtype, leaves through LDS. In the MFMA layout a lane holds 4
// consecutive d of one row per 16-byte chunk, so a direct store instruction
// would touch 32 rows with 8 bytes each; re-read from LDS, a lane holds one
// whole 16-byte chunk and a store instruction writes 64 / (D/8) consecutive
// whole rows. Chunks are XOR-swizzled by row so the writes and re-reads are
// free of bank conflicts. stg is the caller's own 32·D·2-byte LDS region,
// which no other wave touches. l_run is this lane's partial row sum (the
// lane 32 apart holds the rest), m_run the row's running max of
// u = q·k + mask/scale.
// The row block's ticket word (fused split tail): one per (batch, head group,
// m-block), shared by that block's splits; ti as tile_index returns it.
template <int BM, class PT>
__device__ __forceinline__ int ticket_of(PT& p, const TileIdx& ti) {
  const int ng = p.h / p.pack;
  return (ti.b * ng + ti.h / p.pack) * p.num_m + ti.m0 / (BM / p.pack);
}

template <int D, bool BF16, bool SPLIT>
__device__ __forceinline__ void write_rows(const KParams& p, const f32x16 (&oacc)[D / 32], float l_run,
                                           float m_run, int b, int h, int split, int qrow, uint8_t* stg,
                                           int lane) {
  constexpr int DB = D / 32;
  const int l32 = lane & 31, g = lane >> 5;
  const float l = xhalf_sum(l_run);
  const float inv = (l == 0.f || l != l) ? 1.f : 1.f / l;
  constexpr int CH = D / 8;      // 16-byte chunks per row
  constexpr int RPI = 64 / CH;   // rows per re-read instruction
  typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
  typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      f32x4 v4;
#pragma unroll
      for (int i = 0; i < 4; ++i) v4[i] = oacc[db][q4 * 4 + i] * inv;
      u32x2 packed;
      if constexpr (BF16) packed = bitcast<u32x2>(__builtin_convertvector(v4, bf16x4));
      else packed = bitcast<u32x2>(__builtin_convertvector(v4, f16x4));
      const int c = db * 4 + q4;   // chunk of d = db·32 + q4·8 .. +7; this lane's half g
      *reinterpret_cast<u32x2*>(stg + l32 * D * 2 + ((c ^ (l32 & (CH - 1))) * 16) + g * 8) = packed;
    }
  }
  const int ch = lane % CH, r0 = lane / CH;
  const int row0 = qrow - l32;   // the first of the 32 rows
  if constexpr (!SPLIT) {
    const rsrc_t ro = make_rsrc(p.o + (int64_t)b * p.o_bs + (int64_t)h * p.o_hs,
                                (uint32_t)p.sq * p.o_rs * 2u);
#pragma unroll
    for (int k = 0; k < 32 / RPI; ++k) {
      const int r = r0 + k * RPI;
      const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * D * 2 + ((ch ^ (r & (CH - 1))) * 16));
      // rows at or past Sq fall outside the buffer and are dropped
      __builtin_amdgcn_raw_buffer_store_b128(v, ro, (uint32_t)((row0 + r) * p.o_rs + ch * 8) * 2u, 0, 0);
    }
  } else {
    // partial O normalised by the split's own l, rounded to the input
    // dtype as the reference stores it (fa_fwd_launch.h:289-297)
    const int64_t bh = (int64_t)b * p.h + h;
    const int64_t slab = (int64_t)p.b * p.h * p.sq;
    const int64_t pbase = (int64_t)split * slab + bh * p.sq;
    const float lse = (l == 0.f || l != l) ? -INFINITY
                      : __builtin_fmaf(m_run, p.scale, __builtin_amdgcn_logf(l) * 0.69314718f);
    if (p.fuse) {
      // device-scope (sc1) stores: written through to where every XCD reads
      // them, done once this wave's vmcnt drains (the fused tail's release)
      const rsrc_t rp = make_rsrc(p.o_part, p.part_bytes), rl = make_rsrc(p.lse_part, p.lse_bytes);
#pragma unroll
      for (int k = 0; k < 32 / RPI; ++k) {
        const int r = r0 + k * RPI;
        const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * D * 2 + ((ch ^ (r & (CH - 1))) * 16));
        if (row0 + r < p.sq)
          __builtin_amdgcn_raw_buffer_store_b128(v, rp, (uint32_t)(((pbase + row0 + r) * D + ch * 8) * 2), 0,
                                                 kCpolSc1);
      }
      if (g == 0 && qrow < p.sq)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, lse), rl,
                                              (uint32_t)((pbase + qrow) * 4), 0, kCpolSc1);
    } else {
#pragma unroll
      for (int k = 0; k < 32 / RPI; ++k) {
        const int r = r0 + k * RPI;
        const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * D * 2 + ((ch ^ (r & (CH - 1))) * 16));
        if (row0 + r < p.sq) *reinterpret_cast<u32x4*>(p.o_part + (pbase + row0 + r) * D + ch * 8) = v;
      }
      if (g == 0 && qrow < p.sq) p.lse_part[pbase + qrow] = lse;
    }
  }
}

// Memory ordering of the fused split tail (why the last arrival reads every
// split's finished partials, with no fence instruction on either side):
//   * Producer: each wave stores its partial O rows and LSEs with sc1 buffer
//     stores. sc1 is exactly what the compiler emits for an agent-scope
//     relaxed atomic store on gfx950 (global_store ... sc1): the store is
//     written through this XCD's L2 to the level every XCD reads from.
//     wait_vmcnt<0>() then blocks the wave until every one of its stores has
//     been acknowledged (on gfx9 vmcnt counts stores until they complete), and
//     wg_barrier() holds thread 0 until every wave has passed that wait. Only
//     then does thread 0 issue the ticket compare-and-swap.
//   * The ticket word: all arrivals are agent-scope read-modify-writes of one
//     address, so they are totally ordered; the arrival whose count completes
//     the row block has read the value written by every earlier arrival's
//     CAS, each of which was issued after its workgroup's stores completed.
//   * Consumer: the other threads read the LDS flag after a barrier that
//     follows the CAS's return, so no load of the tail issues before the CAS
//     has returned (the GPU does not issue loads speculatively). Every load of
//     shared data (partials, LSEs) is an sc1 buffer load, the instruction the
//     compiler emits for an agent-scope relaxed atomic load: it is served
//     from the device-coherent level, never from a stale line of this XCD's L2.
//   * This is what the compiler's own agent-scope release / acquire lowering
//     provides (buffer_wbl2 sc1 + s_waitcnt vmcnt(0) before the atomic,
//     s_waitcnt vmcnt(0) + buffer_inv sc1 after it) without its whole-cache
//     writeback and invalidate: those exist for plain stores left dirty in L2
//     and plain loads that could hit stale lines, and no plain store or load
//     touches the shared data here. (A release that did the writeback made
//     cfg5 2x slower: every workgroup wrote back its XCD's whole L2.)
//   * The compiler cannot move the stores below the wait or the CAS above the
//     barrier: both helpers end in __atomic_signal_fence(seq_cst), a code
//     motion barrier for memory operations, around side-effecting s_waitcnt /
//     s_barrier builtins. tests/test_isa.py checks the result in the assembly
//     of every split kernel: between its last partial store and the CAS sit
//     s_waitcnt vmcnt(0) and s_barrier in that order, every store in that
//     stretch and every buffer load after the CAS carries sc1.
//   * The argument is about the hardware's order, not the C++ memory model,
//     in which relaxed atomics create no happens-before: the guarantees above
//     are those of the gfx950 instructions the checked assembly contains.
//
// Row-block ticket word: a 48-bit launch tag above a 16-bit arrival count.
// A word holding another tag restarts at 1, so workspace memory left by an
// earlier launch needs no clearing. A graph replays a captured launch with its
// captured tag, so within one tag the count runs on: launch instance k takes
// counts (k-1)·S+1 .. k·S (modulo M = S·floor(65535/S), within 16 bits), and
// the arrival whose count is a multiple of S is the last of its instance.
// Returns the new word.
__device__ __forceinline__ unsigned long long ticket_arrive(unsigned long long* w, unsigned long long tag,
                                                            int S) {
  const unsigned long long M = (unsigned long long)S * (65535u / (unsigned)S);
  unsigned long long old = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), nw;
  do {
    const unsigned long long c = old & 0xffffull;
    nw = ((old >> 16) == tag && c < M) ? old + 1 : ((tag << 16) | 1ull);
  } while (!__hip_atomic_compare_exchange_weak(w, &old, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT));
  return nw;
}
// The count that ends the launch instance an arrival with count c belongs to
__device__ __forceinline__ int ticket_target(int c, int S) { return ((c - 1) / S + 1) * S; }

// Fused split tail, run by every thread of a split workgroup after its rows'
// partials are stored (sc1). Once all of them have completed, one lane counts
// the workgroup in on its row block's ticket; the split that completes the
// count combines the block's rows from every split's partials (sc1 loads, so
// no stale L2 line of this XCD is read), with the combine kernel's arithmetic.
// Nothing waits on another workgroup. flag is one word of LDS no wave is using.
// The row block is recomputed here from the workgroup id. (The compiled
// kernel only: the assembly loops leave no registers for it.)
template <int D, bool BF16, int BM, int NT>
__device__ __forceinline__ void fused_tail(float* tl, const uint8_t* stg_lo, const uint8_t* stg_hi) {
  typedef typename Elt<BF16>::v8 V8;
  constexpr int kS = kFuseMaxSplits;
  static_assert(NT == kS * BM, "one thread per (row, split) LSE");
  uint32_t* flag = reinterpret_cast<uint32_t*>(tl + kS * BM);
  // The kernel's parameters are read here through kernarg_params, not held in
  // SGPRs from the kernel's entry across the tile loop.
  CKParams& p = kernarg_params(*reinterpret_cast<const KParams*>(tl));
  if (!uni(p.fuse)) return;
  const TileIdx tb = tile_index<BM>(p);
  const int ticket = ticket_of<BM>(p, tb), b = tb.b, h0 = tb.h, m0 = tb.m0, own = tb.split;
  wait_vmcnt<0>();
  wg_barrier();
  if (threadIdx.x == 0) {
    const int S = p.num_splits;
    const int c = (int)(ticket_arrive(p.tickets + ticket, p.tag, S) & 0xffffull);
    *flag = (c == ticket_target(c, S)) ? 1u : 0u;
  }
  wg_barrier();
  if (*flag == 0u) return;
  // Block row rr: head h0 + rr / (BM / pack), row m0 + rr % (BM / pack). Its
  // own split's partial is still in the LDS staging of the wave that wrote it
  // (wave j + pack·(m / 32) for head slot j and block-local row m, 32 rows of
  // D elements each, 16-byte units XOR-swizzled by row); the other split's
  // comes by sc1 loads. Weights as in the combine kernel.
  constexpr int CH = D / 8, kTPR = CH, kRPP = NT / kTPR, kPer = BM / kRPP;
  const int S = uni(p.num_splits);
  const int tid = threadIdx.x, c8 = tid % kTPR, rp0 = tid / kTPR;
  const int rows_h = BM / uni(p.pack);
  const int64_t slab = (int64_t)p.b * p.h * p.sq;
  const rsrc_t rpart = make_rsrc_uniform(p.o_part, p.part_bytes);
  const rsrc_t rlse = make_rsrc_uniform(p.lse_part, p.lse_bytes);
  auto grow = [&](int rr, int& h, int& m) {
    h = h0 + rr / rows_h;
    m = m0 + rr % rows_h;
    return ((int64_t)b * p.h + h) * p.sq + m;
  };
  u32x4 raw[kPer][kS];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    int h, m;
    const int64_t row = grow(rp0 + k * kRPP, h, m);
#pragma unroll
    for (int s = 0; s < kS; ++s) {
      const bool in = m < p.sq && s < S && s != own;
      raw[k][s] = __builtin_amdgcn_raw_buffer_load_b128(
          rpart, in ? (uint32_t)(((s * slab + row) * D + c8 * 8) * 2) : 0x80000000u, 0, kCpolSc1);
    }
  }
  {
    const int rr = tid % BM, s = tid / BM;
    int h, m;
    const int64_t row = grow(rr, h, m);
    tl[s * BM + rr] = (m < p.sq && s < S) ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                rlse, (uint32_t)((s * slab + row) * 4), 0, kCpolSc1))
                                          : -INFINITY;
  }
  __syncthreads();
  if (tid < BM) {
    float mx = -INFINITY;
#pragma unroll
    for (int s = 0; s < kS; ++s) mx = fmaxf(mx, tl[s * BM + tid]);
    const float mxc = (mx == -INFINITY) ? 0.f : mx;
    float w[kS], sum = 0.f;
#pragma unroll
    for (int s = 0; s < kS; ++s) {
      w[s] = __builtin_amdgcn_exp2f((tl[s * BM + tid] - mxc) * kLog2e);
      sum += w[s];
    }
    const float inv = (sum > 0.f) ? 1.f / sum : 0.f;
#pragma unroll
    for (int s = 0; s < kS; ++s) tl[s * BM + tid] = w[s] * inv;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int rr = rp0 + k * kRPP;
    int h, m;
    grow(rr, h, m);
    if (m >= p.sq) continue;
    const int j = rr / rows_h, ml = rr % rows_h, wv = j + p.pack * (ml / 32), r32 = ml % 32;
    const uint8_t* st = (wv < 4 ? stg_lo : stg_hi) + (wv & 3) * 32 * D * 2;
    const u32x4 mine = *reinterpret_cast<const u32x4*>(st + r32 * D * 2 + ((c8 ^ (r32 & (CH - 1))) * 16));
    f32x8 acc = {};
#pragma unroll
    for (int s = 0; s < kS; ++s) {
      const float ws = tl[s * BM + rr];
      const u32x4 x = (ws != 0.f) ? (s == own ? mine : raw[k][s]) : u32x4{0u, 0u, 0u, 0u};
      acc += ws * __builtin_convertvector(bitcast<V8>(x), f32x8);
    }
    uint16_t* dst = p.o + (int64_t)b * p.o_bs + (int64_t)h * p.o_hs + (int64_t)m * p.o_rs + c8 * 8;
    *reinterpret_cast<u32x4*>(dst) = bitcast<u32x4>(__builtin_convertvector(acc, V8));
  }
}

template <int D, bool BF16, bool SPLIT, bool MDIRECT, int WAVES>
struct Attn {
  typedef typename Elt<BF16>::v8 V8;
  typedef Geo<D, WAVES> G;
  static constexpr int KD = D / 16;
  static constexpr int DB = D / 32;
  static constexpr int NKB = 2;   // 32-key blocks per tile

  const KParams& p;
  int tid, lane, wave, l32, g;
  const uint16_t *kbase, *vbase, *mbase;
  uint32_t kbytes, vbytes, mbytes;
  rsrc_t rm;
  static constexpr bool mdirect = MDIRECT;
  uint32_t k_off[G::kKWaveLoads];
  uint32_t v_off[G::kKWaveLoads];
  // Mask path. MREG (8 waves, 16-byte aligned rows): each lane loads the 32
  // mask values of its own row straight into registers. Otherwise the tile
  // goes through LDS (sM), loaded with 8 lanes per 128-byte row segment:
  // those grids stream from HBM (4 waves) or read unaligned rows, where the
  // per-row register loads (32 cache lines per instruction) cost more than
  // the LDS round trip.
  static constexpr bool MREG = MDIRECT && WAVES == 8;
  // LDS mask path with bf16 data: the mask can be added on the matrix core
  // (p.mask_mfma): u = A_0·M_0 + A_1·M_1 per 32-key block, where M_c is the
  // 16-key chunk c of the block (keys 16c + 8g .. +7 of the lane's row, the B
  // operand as it sits in LDS) and A_c selects each score's key with weight
  // bf16(1/scale) (A_c[row i][k] = bf16(1/scale) where key π(i) = 16c + k).
  // -inf is first clamped to -max_bf16 (0 × -inf would be NaN); -max·w
  // overflows the fp32 sum back to -inf for w > 1.0078. Masks of 0 and -inf
  // give the same scores as the VALU widening, bit for bit.
  static constexpr bool MMF = BF16 && !MREG;
  bool mmfma = false;
  V8 msel[MMF ? 2 : 1];
  uint32_t m_off[MREG ? 1 : G::kMWaveLoads];
  uint32_t k_rd[KD];
  uint32_t v_rd[DB];
  uint32_t m_rd[4];
  V8 qreg[KD];
  f32x16 oacc[DB];
  f32x16 s[NKB];
  u32x4 mreg[MREG ? 4 : (MDIRECT ? 1 : G::kMWaveLoads)];
  // Scores live in the reference's unscaled domain u = q·k + mask·(1/scale)
  // (csrc/fa/sm89/fa_fwd_kernel.h:286-310); m_run is a max of u, and
  // exp(x - max) = exp2(u·c2 - m_run·c2) with c2 = scale·log2(e) (softmax.h:87).
  float m_run, mlog2, l_run;
  float c2, inv_scale, slack_u;

  __device__ __forceinline__ Attn(const KParams& p_) : p(p_) {}

  __device__ __forceinline__ void init(const TileIdx& ti) {
    tid = threadIdx.x;
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    l32 = lane & 31;
    g = lane >> 5;
    kbase = p.k + (int64_t)ti.b * p.k_bs + (int64_t)ti.hk * p.k_hs;
    vbase = p.v + (int64_t)ti.b * p.v_bs + (int64_t)ti.hk * p.v_hs;
    mbase = p.mask + (int64_t)ti.b * p.m_bs;
    kbytes = (uint32_t)p.sk * p.k_rs * 2u;
    vbytes = (uint32_t)p.sk * p.v_rs * 2u;
    mbytes = (uint32_t)p.msq * p.m_rs * 2u;
    rm = make_rsrc(mbase, mbytes);
#pragma unroll
    for (int i = 0; i < G::kKWaveLoads; ++i) {
      const int u = (i * G::kWaves + wave) * 64 + lane;
      const int r = u / G::kUPR, slot = u % G::kUPR;
      const int key = (r & ~31) + key_perm(r & 31);
      k_off[i] = (uint32_t)(key * p.k_rs + (slot ^ (r % G::kUPR)) * 8) * 2u;
      v_off[i] = (uint32_t)(r * p.v_rs + (slot ^ v_swz<D>(r)) * 8) * 2u;
    }
    if constexpr (MREG) {
      // lane (row l32, half g) holds keys 16g .. 16g+15 of each 32-key block
      m_off[0] = (uint32_t)((ti.m0 + wave * 32 + l32) * p.m_rs + 16 * g) * 2u;
    } else {
#pragma unroll
      for (int i = 0; i < G::kMWaveLoads; ++i) {
        const int u = (wave * G::kMWaveLoads + i) * 64 + lane;   // the wave's own 32 rows
        const int m = u / 8, slot = u % 8;
        m_off[i] = (uint32_t)((ti.m0 + m) * p.m_rs + (slot ^ mask_swz(m)) * 8) * 2u;
      }
      const int mr = wave * 32 + l32;
      mmfma = MMF && uni(p.mask_mfma) != 0;
#pragma unroll
      for (int i = 0; i < 2 * NKB; ++i) {
        // the lane's own keys 16g + 8(i%2) of block i/2, or (matrix-core add)
        // chunk i%2 of the block: keys 16(i%2) + 8g
        const int u = mmfma ? (i / 2) * 4 + 2 * (i % 2) + g : (i / 2) * 4 + 2 * g + (i % 2);
        m_rd[i] = (uint32_t)(mr * kBN + ((u ^ mask_swz(mr)) * 8)) * 2u;
      }
      if constexpr (MMF) {
        const uint32_t sb = (uint32_t)bitcast<uint16_t>((__bf16)(1.f / p.scale));
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int e = key_perm(l32) - 16 * c - 8 * g;
          u32x4 w;
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = (e == 2 * j) ? sb : (e == 2 * j + 1) ? (sb << 16) : 0u;
          msel[c] = bitcast<V8>(w);
        }
      }
    }
    {
      // transpose-read source lane s (in its 16-lane group) reads key row
      // 16g + s/4 (+ a compile-time 32(j/2) + 8(j%2) + 4h), columns
      // 32·db + 16(group%2) + 4(s%4)
      const int s16 = lane & 15, grp = lane >> 4;
      const int row = 16 * g + s16 / 4;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int d = 32 * db + 16 * (grp & 1) + 4 * (s16 & 3);
        v_rd[db] = (uint32_t)(row * D * 2 + (((d / 8) ^ v_swz<D>(row)) * 16) + (d % 8) * 2);
      }
    }
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      const int c = 2 * kd + g;
      k_rd[kd] = (uint32_t)(l32 * G::kUPR + (c ^ (l32 % G::kUPR))) * 16u;
    }
#pragma unroll
    for (int i = 0; i < DB; ++i) oacc[i] = f32x16{};
    m_run = -INFINITY;
    mlog2 = 0.f;
    c2 = p.scale * kLog2e;
    inv_scale = 1.f / p.scale;
    slack_u = kRescaleSlack / p.scale;
    l_run = 0.f;
  }

  __device__ __forceinline__ void load_q(int qrow, rsrc_t rq) {
#pragma unroll
    for (int kd = 0; kd < KD; ++kd)
      qreg[kd] = bitcast<V8>(bload16(rq, (uint32_t)(qrow * p.q_rs + kd * 16 + g * 8) * 2u));
  }

  __device__ __forceinline__ void issue_k(int n, uint16_t* sK) {
    const uint32_t sh = (uint32_t)n * kBN * (uint32_t)p.k_rs * 2u;
    const i32x4 r = make_rsrc_words(reinterpret_cast<const char*>(kbase) + sh, kbytes - sh);
#pragma unroll
    for (int i = 0; i < G::kKWaveLoads; ++i)
      if (p.kv_nt) bload16_lds<true>(r, lds_addr(sK) + (uint32_t)((i * G::kWaves + wave) * 64 * 16), k_off[i]);
      else bload16_lds<false>(r, lds_addr(sK) + (uint32_t)((i * G::kWaves + wave) * 64 * 16), k_off[i]);
  }

  // Mask tile n. MREG: straight into registers, chunk i (8 keys, 16 bytes)
  // holding keys 32(i/2) + 16g + 8(i%2) of the tile (a chunk that starts
  // below Sk ends inside its row: the row stride is a multiple of 8 >= Sk).
  // Otherwise into the wave's own rows of sM: by LDS DMA when rows are
  // 16-byte aligned, else through registers (commit_m stores them), reading
  // chunks that reach past Sk element by element.
  static __device__ __forceinline__ constexpr uint32_t chunk_off(int i) {
    return (uint32_t)(32 * (i / 2) + 8 * (i % 2)) * 2u;
  }
  __device__ __forceinline__ void issue_m(int n, uint16_t* sM) {
    const uint32_t key0 = (uint32_t)n * kBN;
    if constexpr (MREG) {
      const rsrc_t r = make_rsrc(reinterpret_cast<const char*>(mbase) + key0 * 2u, mbytes - key0 * 2u);
#pragma unroll
      for (int i = 0; i < 4; ++i) mreg[i] = bload16(r, m_off[0] + chunk_off(i));
    } else if constexpr (MDIRECT) {
      const i32x4 r = make_rsrc_words(reinterpret_cast<const char*>(mbase) + key0 * 2u, mbytes - key0 * 2u);
#pragma unroll
      for (int i = 0; i < G::kMWaveLoads; ++i)
        bload16_lds(r, lds_addr(sM) + (uint32_t)((wave * G::kMWaveLoads + i) * 64 * 16), m_off[i]);
    } else {
#pragma unroll
      for (int i = 0; i < G::kMWaveLoads; ++i) {
        const int u = (wave * G::kMWaveLoads + i) * 64 + lane;
        const int c = (u % 8) ^ mask_swz(u / 8);
        const int kc = (int)key0 + c * 8;
        const uint32_t off = m_off[i] + key0 * 2u;
        if (kc + 8 <= p.sk) {
          mreg[i] = bload16(rm, off);
        } else {
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t lo = (kc + 2 * j < p.sk)
                ? __builtin_amdgcn_raw_buffer_load_b16(rm, off + 4 * j, 0, 0) : 0u;
            const uint32_t hi = (kc + 2 * j + 1 < p.sk)
                ? __builtin_amdgcn_raw_buffer_load_b16(rm, off + 4 * j + 2, 0, 0) : 0u;
            w[j] = (lo & 0xffffu) | (hi << 16);
          }
          mreg[i] = u32x4{w[0], w[1], w[2], w[3]};
        }
      }
    }
  }

  __device__ __forceinline__ void commit_m(uint16_t* sM) {
    if constexpr (MDIRECT) return;
#pragma unroll
    for (int i = 0; i < G::kMWaveLoads; ++i) {
      const int u = (wave * G::kMWaveLoads + i) * 64 + lane;
      *reinterpret_cast<u32x4*>(sM + u * 8) = mreg[i];
    }
  }

  __device__ __forceinline__ void issue_v(int n, uint16_t* sV) {
    const uint32_t sh = (uint32_t)n * kBN * (uint32_t)p.v_rs * 2u;
    const i32x4 r = make_rsrc_words(reinterpret_cast<const char*>(vbase) + sh, vbytes - sh);
#pragma unroll
    for (int i = 0; i < G::kKWaveLoads; ++i)
      if (p.kv_nt) bload16_lds<true>(r, lds_addr(sV) + (uint32_t)((i * G::kWaves + wave) * 64 * 16), v_off[i]);
      else bload16_lds<false>(r, lds_addr(sV) + (uint32_t)((i * G::kWaves + wave) * 64 * 16), v_off[i]);
  }

  // u = mask·(1/scale) + K·Qᵀ: the widened, pre-scaled mask tile initialises the
  // accumulators, so no pass over the scores is needed between the two GEMMs
  // (the mask work overlaps the MFMAs of the other key block). K operands
  // stream through a window of kWin LDS reads in flight.
  static constexpr int kWin = 2;
  typedef f32x16 Scores[NKB];

  __device__ __forceinline__ void mask_init(const uint16_t* sM) { mask_init(sM, s); }
  __device__ __forceinline__ void mask_init(const uint16_t* sM, Scores& sc) {
    const uint8_t* mb = reinterpret_cast<const uint8_t*>(sM);
    if constexpr (MMF) {
      if (mmfma) {
        typedef unsigned short us2 __attribute__((ext_vector_type(2)));
        const us2 lim = {0xff7fu, 0xff7fu};   // -max_bf16: -inf (0xff80) and above clamp to it
#pragma unroll
        for (int b = 0; b < NKB; ++b) {
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            u32x4 x = *reinterpret_cast<const u32x4*>(mb + m_rd[2 * b + c]);
#pragma unroll
            for (int j = 0; j < 4; ++j)
              x[j] = bitcast<uint32_t>(__builtin_elementwise_min(bitcast<us2>(x[j]), lim));
            sc[b] = Elt<BF16>::mfma(msel[c], bitcast<V8>(x), c == 0 ? f32x16{} : sc[b]);
          }
        }
        return;
      }
    }
#pragma unroll
    for (int b = 0; b < NKB; ++b) {
      u32x4 lo, hi;
      if constexpr (MREG) {
        lo = mreg[2 * b];
        hi = mreg[2 * b + 1];
      } else {
        lo = *reinterpret_cast<const u32x4*>(mb + m_rd[2 * b]);
        hi = *reinterpret_cast<const u32x4*>(mb + m_rd[2 * b + 1]);
      }
      const f32x16 mk = mask_to_f32<BF16>(lo, hi);
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[b][i] = mk[i] * inv_scale;
    }
  }

  __device__ __forceinline__ void qk(const uint16_t* sK) { qk(sK, s); }
  __device__ __forceinline__ void qk(const uint16_t* sK, Scores& sc) {
    const uint8_t* kb8 = reinterpret_cast<const uint8_t*>(sK);
    constexpr int N = NKB * KD;   // step i: local block i / KD, kd = i % KD
    auto rd = [&](int i) {
      return bitcast<V8>(*reinterpret_cast<const u32x4*>(kb8 + (i / KD) * 32 * D * 2 + k_rd[i % KD]));
    };
    V8 win[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) win[i] = rd(i);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const V8 a = win[i % kWin];
      if (i + kWin < N) win[i % kWin] = rd(i + kWin);
      sc[i / KD] = Elt<BF16>::mfma(a, qreg[i % KD], sc[i / KD]);
    }
  }

  // keys past Sk → -inf (only the last tile of a head reaches past Sk)
  __device__ __forceinline__ void apply_tail(int n) { apply_tail(n, s); }
  __device__ __forceinline__ void apply_tail(int n, Scores& sc) {
    if ((n + 1) * kBN > p.sk) {
#pragma unroll
      for (int b = 0; b < NKB; ++b)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = n * kBN + b * 32 + g * 16 + i;
          sc[b][i] = (key < p.sk) ? sc[b][i] : -INFINITY;
        }
    }
  }

  // softmax of tile n and Oᵀ += Vᵀ·Pᵀ, the exponentials of each key step one
  // step ahead of its MFMAs
  // A tile in which no row of the wave has a live key (every score -inf, e.g.
  // outside a sliding window) contributes P = 0 exactly: l and O stay as they
  // are bit for bit, so its exponentials and PV product are skipped.
  __device__ __forceinline__ void softmax_pv(const uint16_t* sVt) {
    if (rescale(s)) exp_pv(sVt, s);
  }

  // row max of a tile's scores; moves the running max (and rescales O, l)
  // only when it grew by more than the slack. Returns whether any row of the
  // wave has a key that is not -inf in this tile (NaN counts as live).
  __device__ __forceinline__ bool rescale(const Scores& sc) {
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < NKB; ++b)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sc[b][i]);
    mx = xhalf_max(mx);
    const bool live = __builtin_amdgcn_ballot_w64(!(mx == -INFINITY)) != 0;
    const bool need = mx > m_run + slack_u;
    if (__builtin_amdgcn_ballot_w64(need)) {
      // lanes that keep their max scale by exactly 1 (also avoids -inf - -inf)
      const float alpha = need ? __builtin_amdgcn_exp2f((m_run - mx) * c2) : 1.f;
      m_run = need ? mx : m_run;
      mlog2 = (m_run == -INFINITY) ? 0.f : m_run * c2;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
    }
    return live;
  }

  // P = exp2(u·c2 − m_run·c2) rounded to the input dtype; l += Σ P; Oᵀ += Vᵀ·Pᵀ.
  // The exponentials of key step j + 1 are issued before the MFMAs of step j,
  // so no MFMA waits on exponentials produced just before it (l accumulates
  // the steps in order either way).
  __device__ __forceinline__ void exp_pv(const uint16_t* sVt, const Scores& sc) {
    // PV operands (step i: local key step j = i / DB of 8 keys, d block
    // db = i % DB) stream through a window of kWin LDS reads in flight.
    constexpr int N = 2 * NKB * DB;
    const uint8_t* vb = reinterpret_cast<const uint8_t*>(sVt);
    auto rd = [&](int i) {
      const int j = i / DB, db = i % DB;
      const int off = ((j / 2) * 32 + (j % 2) * 8) * D * 2;
      const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + v_rd[db] + off));
      const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(vb + v_rd[db] + off + 4 * D * 2));
      return bitcast<V8>(__builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    V8 win[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) win[i] = rd(i);
    auto pstep = [&](int j) {
      f32x8 pf;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pf[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j / 2][(j % 2) * 8 + e], c2, -mlog2));
      return __builtin_convertvector(pf, V8);
    };
    V8 pcur = pstep(0);
    l_run = psum8<BF16>(pcur, l_run);
#pragma unroll
    for (int j = 0; j < 2 * NKB; ++j) {
      V8 pnext;
      if (j + 1 < 2 * NKB) pnext = pstep(j + 1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int i = j * DB + db;
        const V8 a = win[i % kWin];
        if (i + kWin < N) win[i % kWin] = rd(i + kWin);
        oacc[db] = Elt<BF16>::mfma(a, pcur, oacc[db]);
      }
      if (j + 1 < 2 * NKB) {
        l_run = psum8<BF16>(pnext, l_run);
        pcur = pnext;
      }
    }
  }

  __device__ __forceinline__ void epilogue(int b, int h, int split, int qrow, uint8_t* stg) {
    write_rows<D, BF16, SPLIT>(p, oacc, l_run, m_run, b, h, split, qrow, stg, lane);
  }
};

// Software pipeline over KV tiles with NST LDS stages for K and V. Iteration
// over tile n (stage n % NST holds K(n), V(n); the scores already hold
// mask(n)·(1/scale)):
//   [NST = 2: wait for tile n's K/V DMAs] barrier (every wave has landed tile
//   n and left tile n-1's stage); issue mask(n+1) and K(n+NST-1) into tile
//   n-1's stage (8 waves: K after the QK); u += K(n)·Qᵀ; issue V(n+NST-1);
//   softmax(n) fused with Oᵀ += Vᵀ(n)·Pᵀ(n); wait until everything but the
//   newest tile's K/V DMAs has landed and widen mask(n+1) into the scores.
//   One barrier per tile.
// Each wave loads and reads only its own 32 mask rows, so the mask needs one
// LDS buffer and no barrier, and the next tile's GEMM starts right after the
// barrier. Aligned rows arrive by LDS DMA; unaligned rows go through registers
// (element-wise past Sk) and the wave stores them to its rows of the buffer.
// Measured and not kept: testing the mask block before QK to skip a whole
// dead tile, persistent workgroups with cross-item prefetch, a software-
// pipelined softmax(n) / PV(n-1) loop, 4 waves of 64 rows, a combine done by
// each row block's last split (its device-scope release writes back the L2).
#ifndef MI355_FA_STAGES8
#define MI355_FA_STAGES8 2
#endif
#ifndef MI355_FA_STAGES4
#define MI355_FA_STAGES4 2
#endif
// Two waves per SIMD: the 8-wave workgroup alone, or two 4-wave workgroups
// (80 KiB of LDS each at two stages) sharing a CU. DEEP (4 waves, grids of at
// most one workgroup per CU): a third K/V stage, in dynamic LDS, so the
// compiler still budgets registers for two waves per SIMD (static LDS past
// 80 KiB would lift that target and cost AGPR copies in the tile loop).
template <int D, bool BF16, bool SPLIT, bool MDIRECT, int WAVES, bool DEEP, bool MAPONLY = false>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fa_fwd_kernel(const KParams p) {
  typedef Geo<D, WAVES> G;
  typedef Attn<D, BF16, SPLIT, MDIRECT, WAVES> A;
  constexpr int NST = WAVES == 8 ? MI355_FA_STAGES8
                                 : (DEEP && MI355_FA_STAGES4 < 3 ? 3 : MI355_FA_STAGES4);
  static_assert(NST >= 2 && NST <= 4, "two to four stages");
  static_assert(!DEEP || WAVES == 4, "the deep pipeline is a 4-wave variant");
  constexpr int NSS = DEEP ? 2 : NST;   // stages in static LDS; the rest follow in dynamic LDS
  __shared__ __align__(16) uint16_t sKs[NSS][G::kKElems];
  __shared__ __align__(16) uint16_t sVs[NSS][G::kVElems];
  extern __shared__ __align__(16) uint16_t fa_dyn_lds[];   // DEEP: [K stage | V stage] per extra stage
  auto KS = [&](int i) -> uint16_t* {
    return i < NSS ? sKs[i] : fa_dyn_lds + (i - NSS) * (G::kKElems + G::kVElems);
  };
  auto VS = [&](int i) -> uint16_t* {
    return i < NSS ? sVs[i] : fa_dyn_lds + (i - NSS) * (G::kKElems + G::kVElems) + G::kKElems;
  };
  __shared__ __align__(16) uint16_t sM[A::MREG ? 8 : G::kMElems];
  // fused split tail: per (split, row) LSEs then weights, and the ticket flag.
  // 4 waves: in the V stages, which the output staging leaves free. An array
  // of its own would take the workgroup past 80 KiB of LDS, so two could no
  // longer share a CU and the compiler, no longer held to two waves per SIMD,
  // would spend registers past 256 (and AGPR copies in the tile loop).
  constexpr bool kTailOwn = SPLIT && WAVES == 8;
  constexpr int kTailFloats = kFuseMaxSplits * G::kBM + 4;
  static_assert(kTailOwn || !SPLIT || kTailFloats * 4 <= NSS * G::kVElems * 2, "tail fits in the V stages");
  __shared__ __align__(16) float sTail[kTailOwn ? kTailFloats : 1];

  // Live ranges from the live-tile map or the probe and scan: both in one
  // kernel, but the 4-wave deep ones on the LDS-DMA mask path, whose SGPRs
  // the two together would push into spills, have one instance each
  // (MAPONLY: the map, launched when the launch has one)
  constexpr bool kMap = MAPONLY || !MDIRECT || WAVES == 8 || !DEEP;
  constexpr bool kScan = !MAPONLY;
  TileIdx ti = tile_index<G::kBM>(p);
  const TileIdx tg = ti;   // the workgroup's first head and row
  const LiveProbe lp = live_probe<G::kThreads, kMap, kScan, SPLIT>(tg, p);
  place_wave(ti, p, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), 32);
  A a(p);
  a.init(ti);
  int nb = ti.nb, ne = ti.ne;
  const rsrc_t rq = make_rsrc(p.q + (int64_t)ti.b * p.q_bs + (int64_t)ti.h * p.q_hs,
                              (uint32_t)p.sq * p.q_rs * 2u);
  const int qrow = ti.m0 + a.wave * 32 + a.l32;
  // With Sk % 64 != 0, zero the V buffers once: a V row the tail's DMA leaves
  // unwritten then holds 0 or an earlier tile's finite values, and its P is 0,
  // so it adds nothing. Whole tiles overwrite every row: no zeroing, and no
  // barrier before the first DMAs.
  if (p.sk % kBN != 0) {
    for (int i = threadIdx.x; i < G::kVElems / 8; i += G::kThreads)
#pragma unroll
      for (int st = 0; st < NST; ++st) reinterpret_cast<u32x4*>(VS(st))[i] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
  }
  int cnt = ne - nb;
  auto first_tiles = [&]() {
    if (cnt > 0) a.issue_m(nb, sM);
#pragma unroll
    for (int j = 0; j < NST - 1; ++j) {
      if (j < cnt) {
        a.issue_k(nb + j, KS(j));
        a.issue_v(nb + j, VS(j));
      }
    }
  };
  first_tiles();
  a.load_q(qrow, rq);
  wait_vmcnt<0>();   // Q, the first tiles and the live probe, on every path into the loop
  {
    // the last K stage is not loaded before the loop's first barrier
    TileIdx tn = tg;
    if (narrow_to_live<BF16, G::kThreads, G::kBM, 8, true, kMap, kScan, SPLIT>(tn, p, G::kBM / p.pack, lp,
                                                       reinterpret_cast<uint32_t*>(KS(NST - 1)))) {
      // the range moved: the first tiles again, for its first tile
      nb = tn.nb;
      ne = tn.ne;
      cnt = ne - nb;
      first_tiles();
      wait_vmcnt<0>();
    }
  }
  if (cnt > 0) {
    a.commit_m(sM);
    a.mask_init(sM);
  }

  // Loads of one iteration, in issue order: the mask's, then K's, then V's.
  constexpr int kKVLoads = 2 * G::kKWaveLoads;
  auto iter = [&](auto stc, int n) {
    constexpr int ST = decltype(stc)::value;   // (n - nb) % NST
    constexpr int SF = (ST + NST - 1) % NST;   // stage of tile n + NST - 1 (= n - 1)
    const bool more = n + 1 < ne, far = n + NST - 1 < ne;
    if constexpr (NST == 2) wait_vmcnt<0>();
    // A register mask can leave before the barrier (its registers were freed
    // by the previous mask_init); the last tile reloads its own mask (unused)
    // so the loop body has no branch there. An LDS mask waits for the barrier.
    if constexpr (A::MREG) a.issue_m(more ? n + 1 : n, sM);
    wg_barrier();
    if constexpr (!A::MREG) {
      if (more) a.issue_m(n + 1, sM);
    }
    // 4 waves (small grids, HBM streams): K(n+NST-1) goes out before QK(n),
    // for the longest lead. 8 waves (MFMA-bound): after it, so QK's K-operand
    // reads do not share the LDS with the incoming K tile (cfg2 -1.4 %,
    // cfg5 -3.5 %; measured +3 % on cfg4 in the 4-wave kernel).
    if constexpr (WAVES == 4) {
      if (far) a.issue_k(n + NST - 1, KS(SF));
    }
    a.qk(KS(ST));
    if constexpr (WAVES == 8) {
      if (far) a.issue_k(n + NST - 1, KS(SF));
    }
    if (far) a.issue_v(n + NST - 1, VS(SF));
    a.apply_tail(n);
    a.softmax_pv(VS(ST));
    if constexpr (A::MREG) {
      // widen mask(n + 1) into the accumulators (the compiler waits for its
      // loads, and with them for the K/V DMAs issued later). Kept inside this
      // iteration: hoisted past the next barrier it would hold mask(n + 1)'s
      // registers across mask(n + 2)'s loads.
      a.mask_init(sM);
      __builtin_amdgcn_sched_barrier(0);
    } else if (more) {
      if (far) wait_vmcnt<kKVLoads>();
      else wait_vmcnt<0>();
      a.commit_m(sM);
      a.mask_init(sM);
    }
  };
  // Unrolled by NST so every stage index is a compile-time constant; the
  // remainder runs stages 0, 1, ... in order.
  typedef std::integral_constant<int, 0> S0;
  typedef std::integral_constant<int, 1> S1;
  typedef std::integral_constant<int, 2> S2;
  typedef std::integral_constant<int, 3> S3;
  int n = nb;
  for (; n + NST - 1 < ne; n += NST) {
    iter(S0{}, n);
    iter(S1{}, n + 1);
    if constexpr (NST > 2) iter(S2{}, n + 2);
    if constexpr (NST > 3) iter(S3{}, n + 3);
  }
  if (n < ne) iter(S0{}, n);
  if constexpr (NST > 2) {
    if (n + 1 < ne) iter(S1{}, n + 1);
  }
  if constexpr (NST > 3) {
    if (n + 2 < ne) iter(S2{}, n + 2);
  }

  // The K/V stages are free once every wave is past its last tile (and no
  // DMA is in flight): each wave stages its output rows in a private slice.
  static_assert(4 * 32 * D * 2 <= NSS * G::kKElems * 2 && 4 * 32 * D * 2 <= NSS * G::kVElems * 2,
                "output staging fits in the K and V stages");
  wait_vmcnt<0>();
  wg_barrier();
  uint8_t* stg = (a.wave < 4 ? reinterpret_cast<uint8_t*>(KS(0)) : reinterpret_cast<uint8_t*>(VS(0)))
                 + (a.wave & 3) * 32 * D * 2;
  a.epilogue(ti.b, ti.h, ti.split, qrow, stg);
  if constexpr (SPLIT)
    fused_tail<D, BF16, G::kBM, G::kThreads>(kTailOwn ? sTail : reinterpret_cast<float*>(VS(0)),
                                             reinterpret_cast<const uint8_t*>(KS(0)),
                                             reinterpret_cast<const uint8_t*>(VS(0)));
}

// ── software-pipelined tile loop in generated assembly (d = 128) ─────────────
// fa_fwd_kernel_asm<NH>: workgroups of BM = 256 query rows (the 8-wave plan's
// grid), each wave 32·NH rows as NH halves of 32:
//   NH = 1: 8 waves, two per SIMD (256 registers each)
//   NH = 2: 4 waves, one per SIMD (512 registers each; each K and V operand
//           read from LDS then feeds two MFMAs)
// Q and O live in AGPRs. The tile loop is one inline-assembly block generated
// by gen_fa_loop.py (fa_loop.inc), which also emits the operand bindings. It
// runs QK of tile n+1 and PV of tile n as one MFMA stream under the exponentials
// and P conversion of tile n and the mask add, row max and rescale test of tile
// n+1, with all LDS operand reads in one queue. K, V and the mask tile (the
// wave's own rows) arrive by LDS DMA, two stages each, one barrier per tile.
// bf16 masks are added on the matrix core (an MFMA whose A operand selects each
// score's key with weight bf16(1/scale)); fp16 masks by v_fma_mix.
// Masks must have 16-byte aligned rows (the LDS DMA path).
#include "fa_loop.inc"

constexpr int kAsmKStage = 16384;                           // K or V stage: 64 keys x 128 d x 2
constexpr int kAsmMStage = 32768;                           // mask stage: 256 rows x 64 keys x 2
constexpr int kAsmLds = 4 * kAsmKStage + 2 * kAsmMStage;    // 128 KiB
constexpr int kAsmVBase = 2 * kAsmKStage;
constexpr int kAsmMBase = 4 * kAsmKStage;

typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x32 __attribute__((ext_vector_type(32)));
template <int N> struct U32Vec;
template <> struct U32Vec<2> { typedef u32x2 type; };
template <> struct U32Vec<4> { typedef u32x4 type; };
template <> struct U32Vec<8> { typedef u32x8 type; };

template <int NH, bool BF16, bool SPLIT>
__global__ __launch_bounds__(NH == 1 ? 512 : 256)
__attribute__((amdgpu_waves_per_eu(NH == 1 ? 2 : 1, NH == 1 ? 2 : 1)))
void fa_fwd_kernel_asm(const KParams p) {
  constexpr int D = 128;
  constexpr int UPR = D / 8;                       // 16-byte units per K/V row
  constexpr int WAVES = NH == 1 ? 8 : 4;
  constexpr int NKL = 16 / WAVES;                  // K (and V) DMA loads per wave per tile
  constexpr int NML = 4 * NH;                      // mask DMA loads per wave per tile
  constexpr int ROWS = 32 * NH;                    // query rows per wave
  __shared__ __align__(16) uint8_t smem[kAsmLds];
  TileIdx ti = tile_index<256>(p);
  {
    // before the set-up below: its values would be live across the scan, and
    // the registers the scan needs on top of them would spill
    const LiveProbe lp = live_probe<64 * WAVES>(ti, p);
    narrow_to_live<BF16, 64 * WAVES, 256, 4, false>(ti, p, 256 / p.pack, lp, reinterpret_cast<uint32_t*>(smem + kAsmMBase));
  }
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  place_wave(ti, p, wave, ROWS);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;

  const uint16_t* kbase = p.k + (int64_t)ti.b * p.k_bs + (int64_t)ti.hk * p.k_hs;
  const uint16_t* vbase = p.v + (int64_t)ti.b * p.v_bs + (int64_t)ti.hk * p.v_hs;
  const uint16_t* mbase = p.mask + (int64_t)ti.b * p.m_bs;
  const uint32_t kbytes = (uint32_t)p.sk * p.k_rs * 2u, vbytes = (uint32_t)p.sk * p.v_rs * 2u;
  const uint32_t mbytes = (uint32_t)p.msq * p.m_rs * 2u;

  // DMA sources: K rows permuted within 32-key blocks (a lane of the score
  // tile then owns 16 consecutive keys), V in key order, this wave's mask rows
  typename U32Vec<NKL>::type koff, voff;
#pragma unroll
  for (int i = 0; i < NKL; ++i) {
    const int u = (i * WAVES + wave) * 64 + lane;
    const int r = u / UPR, slot = u % UPR;
    const int key = (r & ~31) + key_perm(r & 31);
    koff[i] = (uint32_t)(key * p.k_rs + (slot ^ (r % UPR)) * 8) * 2u;
    voff[i] = (uint32_t)(r * p.v_rs + (slot ^ v_swz<D>(r)) * 8) * 2u;
  }
  typename U32Vec<NML>::type moff;
#pragma unroll
  for (int i = 0; i < NML; ++i) {
    const int m = i * 8 + lane / 8, slot = lane % 8;
    moff[i] = (uint32_t)((ti.m0 + wave * ROWS + m) * p.m_rs + (slot ^ mask_swz(m)) * 8) * 2u;
  }
  u32x8 krd;
#pragma unroll
  for (int i = 0; i < 8; ++i) krd[i] = lds0 + (uint32_t)(l32 * UPR + ((2 * i + g) ^ (l32 % UPR))) * 16u;
  u32x4 vrd, mrd;
  {
    const int s16 = lane & 15, grp = lane >> 4;
    const int row = 16 * g + s16 / 4;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int d = 32 * db + 16 * (grp & 1) + 4 * (s16 & 3);
      vrd[db] = lds0 + kAsmVBase + (uint32_t)(row * D * 2 + (((d / 8) ^ v_swz<D>(row)) * 16) + (d % 8) * 2);
    }
    // mask read i of block b = i / 2: bf16 reads chunk c = i % 2 (keys 16c + 8g ..
    // +7, the B operand of a mask MFMA); fp16 reads the lane's own 16 keys
    // 16g .. +15 as two 8-key units (widened by v_fma_mix). Half h adds 4096.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = BF16 ? 4 * (i / 2) + 2 * (i % 2) + g : 4 * (i / 2) + 2 * g + (i % 2);
      mrd[i] = lds0 + kAsmMBase + (uint32_t)(wave * ROWS * 128 + l32 * 128 + ((c ^ mask_swz(l32)) * 16));
    }
  }
  // bf16 mask selectors: A_c[row i][k] = bf16(1/scale) where key π(i) = 16c + k
  // (this lane: row l32, k = 8g + e), else 0
  u32x8 msel = {};
  if constexpr (BF16) {
    const uint32_t sb = (uint32_t)bitcast<uint16_t>((__bf16)(1.f / p.scale));
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int e = key_perm(l32) - 16 * c - 8 * g;
#pragma unroll
      for (int w = 0; w < 4; ++w) msel[4 * c + w] = (e == 2 * w) ? sb : (e == 2 * w + 1) ? (sb << 16) : 0u;
    }
  }
  const uint32_t mclamp = __builtin_amdgcn_readfirstlane(0xff7fff7fu);   // -max_bf16 pair
  // Q of every half (rows past Sq read 0)
  const rsrc_t rq = make_rsrc(p.q + (int64_t)ti.b * p.q_bs + (int64_t)ti.h * p.q_hs,
                              (uint32_t)p.sq * p.q_rs * 2u);
  u32x32 q[NH];
#pragma unroll
  for (int hh = 0; hh < NH; ++hh) {
    const int qrow = ti.m0 + wave * ROWS + hh * 32 + l32;
#pragma unroll
    for (int kd = 0; kd < 8; ++kd) {
      const u32x4 v = bload16(rq, (uint32_t)(qrow * p.q_rs + kd * 16 + g * 8) * 2u);
#pragma unroll
      for (int e = 0; e < 4; ++e) q[hh][4 * kd + e] = v[e];
    }
  }
  // With Sk % 64 != 0 the last tile's DMA leaves V rows unwritten: zero the
  // V stages once so those rows hold finite values (their P is exactly 0).
  if (p.sk % kBN != 0) {
    for (int i = tid; i < 2 * kAsmKStage / 16; i += 64 * WAVES)
      reinterpret_cast<u32x4*>(smem + kAsmVBase)[i] = u32x4{0u, 0u, 0u, 0u};
  }
  wait_vmcnt<0>();
  __syncthreads();
  const int nb = ti.nb, ne = ti.ne;
  const int cnt = ne - nb;

  const uint32_t ksh = (uint32_t)nb * kBN * (uint32_t)p.k_rs * 2u;
  const uint32_t vsh = (uint32_t)nb * kBN * (uint32_t)p.v_rs * 2u;
  const uint32_t msh = (uint32_t)nb * kBN * 2u;
  const uint64_t ka = reinterpret_cast<uint64_t>(kbase) + ksh;
  const uint64_t va = reinterpret_cast<uint64_t>(vbase) + vsh;
  const uint64_t ma = reinterpret_cast<uint64_t>(mbase) + msh;
  // Integer scalars go through readfirstlane (SGPR operands). The float
  // scalars, which the compiler computes in VGPRs, are bound to fixed VGPRs
  // outside the loop's working set (handed to an "s" operand they arrive as
  // whatever VGPR holds them, possibly inside the loop's register range).
  auto sgpr = [](uint32_t x) { return __builtin_amdgcn_readfirstlane(x); };
  const uint32_t klo = sgpr((uint32_t)ka), khi = sgpr((uint32_t)(ka >> 32) & 0xffffu);
  const uint32_t kn = sgpr(kbytes - ksh);
  const uint32_t vlo = sgpr((uint32_t)va), vhi = sgpr((uint32_t)(va >> 32) & 0xffffu);
  const uint32_t vn = sgpr(vbytes - vsh);
  const uint32_t mlo = sgpr((uint32_t)ma), mhi = sgpr((uint32_t)(ma >> 32) & 0xffffu);
  const uint32_t mn = sgpr(mbytes - msh);
  const uint32_t fl = sgpr((uint32_t)kRsrcFlags);
  const uint32_t kstep = sgpr((uint32_t)kBN * p.k_rs * 2u);
  const uint32_t vstep = sgpr((uint32_t)kBN * p.v_rs * 2u);
  const uint32_t lds_k = sgpr(lds0 + (uint32_t)wave * 1024u);
  const uint32_t lds_v = sgpr(lds0 + kAsmVBase + (uint32_t)wave * 1024u);
  const uint32_t lds_m = sgpr(lds0 + kAsmMBase + (uint32_t)(wave * ROWS * 128));
  const uint32_t lim = sgpr((ne == p.num_n && p.sk % kBN) ? (uint32_t)(p.sk % kBN) : 64u);
  const float c2 = p.scale * kLog2e, inv_scale = 1.f / p.scale, slack = kRescaleSlack / p.scale;
  const float neginf = -INFINITY;
  const uint32_t ntiles = sgpr((uint32_t)cnt);

  f32x16 o[4 * NH];
  float mrun[NH], lsum[NH];
  if (cnt > 0) {
    if constexpr (NH == 2) {
      if constexpr (BF16) asm volatile(MI355_W64_LOOP_BF16 : MI355_W64_OUTPUTS_BF16 : MI355_W64_INPUTS_BF16 : MI355_W64_CLOBBERS_BF16);
      else asm volatile(MI355_W64_LOOP_F16 : MI355_W64_OUTPUTS_F16 : MI355_W64_INPUTS_F16 : MI355_W64_CLOBBERS_F16);
    } else {
      if constexpr (BF16) asm volatile(MI355_W32_LOOP_BF16 : MI355_W32_OUTPUTS_BF16 : MI355_W32_INPUTS_BF16 : MI355_W32_CLOBBERS_BF16);
      else asm volatile(MI355_W32_LOOP_F16 : MI355_W32_OUTPUTS_F16 : MI355_W32_INPUTS_F16 : MI355_W32_CLOBBERS_F16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4 * NH; ++i) o[i] = f32x16{};
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) { mrun[hh] = -INFINITY; lsum[hh] = 0.f; }
  }
  // every wave is past its last LDS read and DMA: LDS becomes output staging
  wait_vmcnt<0>();
  wg_barrier();
#pragma unroll
  for (int hh = 0; hh < NH; ++hh) {
    const f32x16 oh[4] = {o[4 * hh], o[4 * hh + 1], o[4 * hh + 2], o[4 * hh + 3]};
    const int qrow = ti.m0 + wave * ROWS + hh * 32 + l32;
    write_rows<D, BF16, SPLIT>(p, oh, lsum[hh], mrun[hh], ti.b, ti.h, ti.split, qrow,
                               smem + (wave * NH + hh) * 8192, lane);
  }
}

// ── ping-pong tile loop in generated assembly (bf16, d = 128) ────────────────
// fa_fwd_kernel_pp: 8 waves of 32 query rows; waves 0-3 and 4-7 run the same
// phases one phase apart (one workgroup barrier between phases), so on every
// SIMD one wave issues an MFMA phase (mask, QK(t), PV(t-1)) while its partner
// issues a VALU phase (max, exponentials, P, row sums of its tile). K and V
// have three LDS stages, the mask two (160 KiB); waves 0-3 issue all K/V DMA.
// The loop is MI355_PP_LOOP_BF16 from gen_fa_loop.py.
constexpr int kPpKStage = 16384;
constexpr int kPpVBase = 3 * kPpKStage;
constexpr int kPpMBase = 6 * kPpKStage;
constexpr int kPpLds = kPpMBase + 2 * 32768;    // 160 KiB

// MAPPED: the live ranges come from the live-tile map (a launch that has
// one), else from the probe and scan; the two are separate instances because
// both in one push the prologue's SGPRs past what the allocator can spill.
template <bool SPLIT, bool MAPPED>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fa_fwd_kernel_pp(const KParams p) {
  constexpr int D = 128;
  constexpr int UPR = D / 8;
  __shared__ __align__(16) uint8_t smem[kPpLds];
  TileIdx ti = tile_index<256>(p);
  if constexpr (MAPPED) {
    if (uni(kernarg_params(p).live)) range_from_map_wave(ti, kernarg_params(p), 256 / p.pack);
  } else {
    // before the set-up below: its values would be live across the scan, and
    // the SGPRs the scan needs on top of them would spill
    const LiveProbe lp = live_probe<512>(ti, p);
    narrow_to_live<true, 512, 256, 4, false>(ti, p, 256 / p.pack, lp, reinterpret_cast<uint32_t*>(smem + kPpMBase));
  }
  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  place_wave(ti, p, wave, 32);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  const uint16_t* kbase = p.k + (int64_t)ti.b * p.k_bs + (int64_t)ti.hk * p.k_hs;
  const uint16_t* vbase = p.v + (int64_t)ti.b * p.v_bs + (int64_t)ti.hk * p.v_hs;
  const uint16_t* mbase = p.mask + (int64_t)ti.b * p.m_bs;
  const uint32_t kbytes = (uint32_t)p.sk * p.k_rs * 2u, vbytes = (uint32_t)p.sk * p.v_rs * 2u;
  const uint32_t mbytes = (uint32_t)p.msq * p.m_rs * 2u;
  const int wa = wave & 3;   // position within the group (group A issues K/V)

  // K/V DMA sources of group-A wave wa, loads i = 0, 1: unit u = wa·64 + lane
  // of a 16-row slice, row r = u/16 + 16i of the 64-key tile (keys π-permuted
  // per 32); loads 2 and 3 read the same offsets through descriptors 32 rows on
  u32x2 koff, voff;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int u = wa * 64 + lane;
    const int r = u / UPR + 16 * i, slot = u % UPR;
    const int key = (r & ~31) + key_perm(r & 31);
    koff[i] = (uint32_t)(key * p.k_rs + (slot ^ (r % UPR)) * 8) * 2u;
    voff[i] = (uint32_t)(r * p.v_rs + (slot ^ v_swz<D>(r)) * 8) * 2u;
  }
  u32x2 moff;   // this wave's mask rows: 8 per load (loads 2 and 3: 16 rows on, by descriptor)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = i * 8 + lane / 8, slot = lane % 8;
    moff[i] = (uint32_t)((ti.m0 + wave * 32 + m) * p.m_rs + (slot ^ mask_swz(m)) * 8) * 2u;
  }
  u32x8 krd;
#pragma unroll
  for (int i = 0; i < 8; ++i) krd[i] = lds0 + (uint32_t)(l32 * UPR + ((2 * i + g) ^ (l32 % UPR))) * 16u;
  u32x4 vrd, mrd;
  {
    const int s16 = lane & 15, grp = lane >> 4;
    const int row = 16 * g + s16 / 4;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int d = 32 * db + 16 * (grp & 1) + 4 * (s16 & 3);
      vrd[db] = lds0 + kPpVBase + (uint32_t)(row * D * 2 + (((d / 8) ^ v_swz<D>(row)) * 16) + (d % 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 4 * (i / 2) + 2 * (i % 2) + g;
      mrd[i] = lds0 + kPpMBase + (uint32_t)(wave * 32 * 128 + l32 * 128 + ((c ^ mask_swz(l32)) * 16));
    }
  }
  u32x8 msel = {};
  {
    const uint32_t sb = (uint32_t)bitcast<uint16_t>((__bf16)(1.f / p.scale));
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int e = key_perm(l32) - 16 * c - 8 * g;
#pragma unroll
      for (int w = 0; w < 4; ++w) msel[4 * c + w] = (e == 2 * w) ? sb : (e == 2 * w + 1) ? (sb << 16) : 0u;
    }
  }
  // Q goes straight from HBM into the loop's AGPRs (the loop issues those
  // loads with its first tiles' DMA): its buffer and this lane's row offset
  const uint64_t qa = reinterpret_cast<uint64_t>(p.q + (int64_t)ti.b * p.q_bs + (int64_t)ti.h * p.q_hs);
  uint32_t qoff = (uint32_t)((ti.m0 + wave * 32 + l32) * p.q_rs + g * 8) * 2u;
  // V rows the last tile's DMA leaves unwritten (Sk % 64) must hold finite
  // values: zeroed before any wave's DMA can land in the V stages
  if (p.sk % kBN != 0) {
    for (int i = tid; i < 3 * kPpKStage / 16; i += 512)
      reinterpret_cast<u32x4*>(smem + kPpVBase)[i] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
  }
  const int nb = ti.nb, ne = ti.ne, cnt = ne - nb;

  const uint32_t ksh = (uint32_t)nb * kBN * (uint32_t)p.k_rs * 2u;
  const uint32_t vsh = (uint32_t)nb * kBN * (uint32_t)p.v_rs * 2u;
  const uint32_t msh = (uint32_t)nb * kBN * 2u;
  const uint64_t ka = reinterpret_cast<uint64_t>(kbase) + ksh;
  const uint64_t va = reinterpret_cast<uint64_t>(vbase) + vsh;
  const uint64_t ma = reinterpret_cast<uint64_t>(mbase) + msh;
  auto sgpr = [](uint32_t x) { return __builtin_amdgcn_readfirstlane(x); };
  // raw buffer descriptor of `bytes` at `base`, `skip` bytes on (size
  // saturating at 0); loads 2 and 3 of each tensor use the second one
  auto desc = [&](uint64_t base, uint32_t bytes, uint32_t skip) {
    const uint64_t b = base + skip;
    return u32x4{(uint32_t)sgpr((uint32_t)b), (uint32_t)sgpr((uint32_t)(b >> 32) & 0xffffu),
                 (uint32_t)sgpr(bytes > skip ? bytes - skip : 0u), (uint32_t)sgpr((uint32_t)kRsrcFlags)};
  };
  u32x4 kd0 = desc(ka, kbytes - ksh, 0), kd1 = desc(ka, kbytes - ksh, 32u * p.k_rs * 2u);
  u32x4 vd0 = desc(va, vbytes - vsh, 0), vd1 = desc(va, vbytes - vsh, 32u * p.v_rs * 2u);
  u32x4 md0 = desc(ma, mbytes - msh, 0), md1 = desc(ma, mbytes - msh, 16u * p.m_rs * 2u);
  const uint32_t kstep = sgpr((uint32_t)kBN * p.k_rs * 2u);
  const uint32_t vstep = sgpr((uint32_t)kBN * p.v_rs * 2u);
  const uint32_t lds_k = sgpr(lds0 + (uint32_t)wa * 1024u);
  const uint32_t lds_v = sgpr(lds0 + (uint32_t)wa * 1024u);   // + kPpVBase in the loop's offsets
  const uint32_t lds_m = sgpr(lds0 + kPpMBase + (uint32_t)(wave * 32 * 128));
  const uint32_t lim = sgpr((ne == p.num_n && p.sk % kBN) ? (uint32_t)(p.sk % kBN) : 64u);
  // host-computed float scalars: kernel arguments, hence SGPRs (a float computed
  // here in VALU and handed to an "s" operand can arrive as a VGPR inside the
  // loop's registers, and an explicit readfirstlane right after the VALU write
  // is a hazard the compiler does not see through inline assembly)
  const uint32_t c2 = p.c2_bits, slack = p.slack_bits;
  const uint32_t neginf = sgpr(0xff800000u);
  const uint32_t mclamp = sgpr(0xff7fff7fu);
  const uint32_t ntiles = sgpr((uint32_t)cnt);
  const uint32_t grp = sgpr((uint32_t)(wave >> 2));
  u32x4 qd = desc(qa, (uint32_t)p.sq * p.q_rs * 2u, 0);

  f32x16 o[4];
  float mrun[1], lsum[1];
  if (cnt > 0) {
    asm volatile(MI355_PP_LOOP_BF16 : MI355_PP_OUTPUTS_BF16 : MI355_PP_INPUTS_BF16 : MI355_PP_CLOBBERS_BF16);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32x16{};
    mrun[0] = -INFINITY;
    lsum[0] = 0.f;
  }
  wait_vmcnt<0>();
  wg_barrier();
  const int qrow = ti.m0 + wave * 32 + l32;
  write_rows<D, true, SPLIT>(p, o, lsum[0], mrun[0], ti.b, ti.h, ti.split, qrow, smem + wave * 8192, lane);
}

// ── split-KV combine ────────────────────────────────────────────────────────
struct CParams {
  const uint16_t* o_part;
  const float* lse_part;
  uint16_t* o;
  int64_t o_bs, o_hs, o_rs;
  int b, h, sq, num_splits;
  int64_t rows;  // B*H*Sq
  uint32_t part_bytes;   // bytes of o_part when below 2^31 (buffer-addressed loads), else 0
};

// Workgroup = kCombineThreads / (D/8) rows × D columns: 256 threads (16 rows
// at d = 128) for large grids, one wave (4 rows) when that would leave fewer
// than 1024 workgroups, so a small split grid still fills the chip; thread = 8
// consecutive d-values of a row (one 16-byte load per split). Phase 1 stages the rows' LSEs in LDS and turns
// them into weights w_s = exp(lse_s − max) / Σ (all-(-inf) row → all weights
// 0 → output 0); phase 2 accumulates Σ w_s·O_s in fp32 with up to 16 (one
// wave) or 8 (256 threads) splits' loads in flight (more spills SGPRs). (Issuing them before phase 1 is slower: loads complete in
// order, so the LSE reads would wait behind them.)
template <int D, bool BF16, int kCombineThreads>
__global__ __launch_bounds__(kCombineThreads) void fa_combine_kernel(const CParams p) {
  typedef typename Elt<BF16>::v8 V8;
  constexpr int kTPR = D / 8;                     // threads per row
  constexpr int kRows = kCombineThreads / kTPR;   // rows per workgroup
  // splits' loads in flight per thread: all of a typical small grid's splits
  // in one round trip for the one-wave variant; 8 keeps the large-grid
  // variant's registers (and occupancy) low
  constexpr int kBatch = kCombineThreads == 64 ? 16 : 8;
  __shared__ float sw[kMaxSplits * kRows];
  const int tid = threadIdx.x;
  const int64_t row0 = (int64_t)blockIdx.x * kRows;
  const int64_t slab = p.rows;
  const int S = p.num_splits;
  // up to 16 splits in the one-wave form, 4 in the 256-thread one
  constexpr int kOnePass = kCombineThreads == 64 ? 16 : 4;
  if (S <= kOnePass && p.part_bytes) {
    // Few splits: each thread loads its row's LSEs and its partial slices
    // together (one round trip instead of the LSE phase's and then the
    // partials') and weighs them itself, no LDS or barrier; the same
    // arithmetic in the same order (bit-identical). cfg5 (2 splits, combine
    // launch after the ping-pong loop): 44.5 -> 43.1 µs hot; cfg4 (16
    // splits, one-wave workgroups): 1-2 µs faster.
    const int r = tid / kTPR, c8 = tid % kTPR;
    const int64_t row = row0 + r;
    if (row >= p.rows) return;
    const rsrc_t rp = make_rsrc(p.o_part, p.part_bytes);
    const uint32_t off0 = (uint32_t)((row * D + c8 * 8) * 2);
    const uint32_t sstep = (uint32_t)(slab * D * 2);
    float l[kOnePass];
    u32x4 raw[kOnePass];
#pragma unroll
    for (int u = 0; u < kOnePass; ++u) {   // past S: lse -inf (weight 0), an out-of-range load (0)
      l[u] = u < S ? p.lse_part[u * slab + row] : -INFINITY;
      raw[u] = bload16(rp, u < S ? off0 + (uint32_t)u * sstep : 0x80000000u);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < kOnePass; ++u) mx = fmaxf(mx, l[u]);
    const float mxc = (mx == -INFINITY) ? 0.f : mx;
    float w[kOnePass], sum = 0.f;
#pragma unroll
    for (int u = 0; u < kOnePass; ++u) {
      w[u] = __builtin_amdgcn_exp2f((l[u] - mxc) * kLog2e);
      sum += w[u];
    }
    const float inv = (sum > 0.f) ? 1.f / sum : 0.f;
    f32x8 acc = {};
#pragma unroll
    for (int u = 0; u < kOnePass; ++u) acc += (w[u] * inv) * __builtin_convertvector(bitcast<V8>(raw[u]), f32x8);
    const int64_t bh = row / p.sq;
    const int m = (int)(row % p.sq);
    const int b = (int)(bh / p.h), h = (int)(bh % p.h);
    uint16_t* dst = p.o + (int64_t)b * p.o_bs + (int64_t)h * p.o_hs + (int64_t)m * p.o_rs + c8 * 8;
    *reinterpret_cast<u32x4*>(dst) = bitcast<u32x4>(__builtin_convertvector(acc, V8));
    return;
  }
  for (int i = tid; i < S * kRows; i += kCombineThreads) {
    const int s = i / kRows, rr = i % kRows;
    const int64_t lrow = row0 + rr;
    sw[i] = (lrow < p.rows) ? p.lse_part[s * slab + lrow] : -INFINITY;
  }
  __syncthreads();
  if (tid < kRows) {
    float mx = -INFINITY;
    for (int s = 0; s < S; ++s) mx = fmaxf(mx, sw[s * kRows + tid]);
    const float mxc = (mx == -INFINITY) ? 0.f : mx;
    float sum = 0.f;
    for (int s = 0; s < S; ++s) {
      const float w = __builtin_amdgcn_exp2f((sw[s * kRows + tid] - mxc) * kLog2e);
      sw[s * kRows + tid] = w;
      sum += w;
    }
    const float inv = (sum > 0.f) ? 1.f / sum : 0.f;
    for (int s = 0; s < S; ++s) sw[s * kRows + tid] *= inv;
  }
  __syncthreads();
  const int r = tid / kTPR;
  const int c8 = tid % kTPR;
  const int64_t row = row0 + r;
  if (row >= p.rows) return;
  const uint16_t* src = p.o_part + row * D + c8 * 8;
  f32x8 acc = {};
  // A split with weight 0 (lse = -inf: no live key of the row in that split,
  // e.g. outside a sliding window) adds exactly nothing, so its partial is not
  // fetched (cf. the active-split mask of csrc/fa/sm89/fa_fwd_kernel.h:1458-1468;
  // here per row). Branch-free: the lane's buffer offset moves past the end
  // of the partials, and an out-of-range buffer load returns 0 without a
  // memory access, keeping every split's load of the batch in flight together.
  if (p.part_bytes) {
    const rsrc_t rp = make_rsrc(p.o_part, p.part_bytes);
    const uint32_t off0 = (uint32_t)((row * D + c8 * 8) * 2);
    const uint32_t sstep = (uint32_t)(slab * D * 2);
    for (int s0 = 0; s0 < S; s0 += kBatch) {
      u32x4 raw[kBatch];
      float w[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        w[u] = (s0 + u < S) ? sw[(s0 + u) * kRows + r] : 0.f;
        raw[u] = bload16(rp, w[u] != 0.f ? off0 + (uint32_t)(s0 + u) * sstep : 0x80000000u);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) acc += w[u] * __builtin_convertvector(bitcast<V8>(raw[u]), f32x8);
    }
  } else {
    for (int s0 = 0; s0 < S; s0 += kBatch) {
      u32x4 raw[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (s0 + u < S) raw[u] = *reinterpret_cast<const u32x4*>(src + (int64_t)(s0 + u) * slab * D);
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (s0 + u < S) acc += sw[(s0 + u) * kRows + r] * __builtin_convertvector(bitcast<V8>(raw[u]), f32x8);
    }
  }
  const int64_t bh = row / p.sq;
  const int m = (int)(row % p.sq);
  const int b = (int)(bh / p.h), h = (int)(bh % p.h);
  uint16_t* dst = p.o + (int64_t)b * p.o_bs + (int64_t)h * p.o_hs + (int64_t)m * p.o_rs + c8 * 8;
  *reinterpret_cast<u32x4*>(dst) = bitcast<u32x4>(__builtin_convertvector(acc, V8));
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
// slots = workgroups resident per CU (cap_fill = slots·SMs / m-blocks; the
// reference's kernel fits 2 per SM). Exported as mi355_fa_cost_model_splits
// with the reference's constants; the launcher's own plan (make_plan) uses an
// occupancy cost model fitted to MI355X timings instead.
static int cost_model_splits(int total_mblocks, int nb, int block_m, int d, int cus,
                             int slots = 2) {
  if (cus <= 0) cus = 1;
  if (total_mblocks <= 0 || nb <= 0) return 1;
  if (total_mblocks >= 0.8f * cus) return 1;
  if (nb <= 4) return 1;
  const float K = (d == 128) ? 2.25f : 2.5f;
  const int combine_units = total_mblocks * (block_m / 32) * (d / 32);
  const float P = fmaxf(0.35f, (float)combine_units / (float)cus);
  const float s_star = sqrtf((float)nb * K / P);
  const int cap_fill = (slots * cus) / total_mblocks > 1 ? (slots * cus) / total_mblocks : 1;
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

// The caller's variant selection (all zero: the library's own choices).
static mi355_fa_variant variant_of(const mi355_fa_params* p) {
  mi355_fa_variant v{};
  if (p->variant) v = *p->variant;
  return v;
}

// MI355_FA_NUM_SPLITS, the one tuning override read from the environment:
// read once per process, 0 when unset or not a positive number.
static int env_num_splits() {
  static const int n = [] {
    const char* e = getenv("MI355_FA_NUM_SPLITS");
    const int v = e ? atoi(e) : 0;
    return v > 0 ? v : 0;
  }();
  return n;
}

struct Plan {
  int waves, block_m, num_m, num_n, splits, n_per_split;
  int pack;   // q-heads per workgroup; block_m / pack rows of each
  int head_major;
  size_t o_part_bytes, lse_bytes, ticket_bytes, ws_bytes;
  int fuse;   // split tail fused into the main kernel (no combine launch)
  int deep;   // 4 waves, at most one workgroup per CU: three K/V stages
  // Generated-assembly loop form for d = 128 8-wave plans with aligned mask
  // rows: 3 = ping-pong (bf16; fp16 runs the 32-row loop), 1 = 32-row loop,
  // 2 = 64-row loop, 0 = the compiled kernel.
  int loop;
  // Live-range narrowing: 2 = the default policy (on for split launches and
  // for the compiled kernel, off for unsplit launches of the assembly loops),
  // 1 = on everywhere, 0 = off.
  int live;
  int mask_mfma_off;   // the compiled kernel widens bf16 masks on the VALU
  int kv_nt;           // every K/V tile is read by one workgroup: non-temporal loads
  int live_map;        // a live-tile map pre-pass serves the live ranges (unaligned mask rows)
  int map_row_bytes, map_slices;
  int64_t map_full_off;
  size_t map_bytes;
  int staged;          // unaligned mask rows copied to an aligned staged mask
  int stage_rs;
  size_t stage_bytes;
};

// Tile plan: the workgroup size (4 or 8 waves) and split count with the
// lowest modelled launch time. The model prices the busiest CU, which runs
// k = ceil(W / CUs) of the W workgroups: 8-wave workgroups (BM = 256) one
// after another; 4-wave workgroups (BM = 128) two at a time (a CU holds
// two), an odd last one alone and faster. Each workgroup costs a fixed part
// plus a per-KV-tile part; a split launch adds the combine (a fixed part,
// its partial bytes and the splits per row). The constants are least-squares
// fits, on relative error, to hot back-to-back timings on MI355X with zero
// masks: d = 128 over 98 shapes (bh 1..64, Sq 1..2048, Sk 1k..32k), d = 64
// over 76, each with both workgroup sizes and 1..64 splits. Chosen that way,
// the plans come within 1 % (d = 128) and 3 % (d = 64) of each shape's
// measured best in total, where filling one round of CUs with 8-wave
// workgroups, else with 4-wave ones, came within 5 % and 10 %. Every split
// keeps >= 4 KV tiles.
struct PlanCost { float t8, o8, t4pair, t4solo, o4, c0, c_mb, c_split; };
constexpr PlanCost kCostD128 = {1.819f, 3.630f, 2.197f, 1.258f, 1.923f, 5.251f, 0.453f, 0.106f};
constexpr PlanCost kCostD64 = {1.334f, 2.139f, 1.427f, 0.932f, 1.109f, 5.791f, 0.417f, 0.128f};

static float plan_cost(const PlanCost& c, int bh, int sq, int num_n, int d, int waves, int s,
                       int cus, int pack = 1) {
  const int64_t wgs = (int64_t)(bh / pack) * ceil_div(sq, 32 * waves / pack) * s;
  const int64_t k = (wgs + cus - 1) / cus;   // workgroups on the busiest CU
  const float nps = (float)ceil_div(num_n, s);
  float t = waves == 8 ? (float)k * (nps * c.t8 + c.o8)
                       : (float)(k / 2) * (nps * c.t4pair + c.o4) + (float)(k % 2) * (nps * c.t4solo + c.o4);
  if (s > 1) t += c.c0 + c.c_mb * ((float)bh * sq * s * d * 2.f * 1e-6f) + c.c_split * (float)s;
  return t;
}

// Heads per workgroup: GQA heads that share a KV head also share the mask
// rows, so packing them makes the waves of one workgroup read the same mask
// rows together. A power of two dividing H / Hk, at most 4 (the 4-wave
// workgroups and the 64-row waves of the 4-wave assembly form hold 4 heads).
static int pick_pack(const mi355_fa_params* p, const mi355_fa_variant& v) {
  const int ratio = p->h / p->h_k;
  int want = 4;
  if (v.pack == 1 || v.pack == 2 || v.pack == 4) want = v.pack;
  int pk = 1;
  while (pk * 2 <= want && ratio % (pk * 2) == 0) pk *= 2;
  return pk;
}

static int order_head_major(const mi355_fa_params* p, const Plan& pl, int cus,
                            const mi355_fa_variant& v) {
  if (v.order == 1) return 1;
  if (v.order == 2) return 0;
  if (v.order == 3) return 2;
  const double R = (double)(cus / 8 > 0 ? cus / 8 : 1) * (pl.waves == 4 ? 2 : 1);   // workgroups per XCD round
  const double G = p->h / pl.pack;                                   // head groups (one K/V head each)
  const double M = ceil_div(p->seqlen_q, pl.block_m / pl.pack);      // m-blocks
  const double S = pl.splits;
  const double kv = (double)p->seqlen_k / S * p->d * 4.0;            // K+V of one group, one split
  const double mk = (double)(pl.block_m / pl.pack) * p->seqlen_k / S * 2.0;   // mask of one m-block, one split
  auto up = [](double a, double b) { return std::ceil(a / b); };
  // m-blocks fastest, then splits, then groups: the round's ids cover
  // ceil(R/M) (group, split) pairs and min(R, M) m-blocks of each split seen
  const double pairs = std::min(up(R, M), S * G);
  const double m_fetch = pairs * kv + std::min(R, M) * std::min(S, pairs) * mk;
  // groups fastest, then m-blocks, then splits: ceil(R/G) (split, m-block)
  // mask pieces and min(R, G) groups of each split seen
  const double h_fetch = std::min(up(R, G), M * S) * mk + std::min(R, G) * std::min(S, up(R, G * M)) * kv;
  // Heads fastest in a split launch: the splits of a row block next, so that
  // every workgroup reading that block's mask rows (its head groups times its
  // splits; each one scans them when the mask has dead edges) runs on one XCD
  // at once (cfg5's shape: 1 % faster on a sliding window and on a dense mask).
  if (h_fetch < m_fetch) return S > 1 ? 2 : 1;
  return 0;
}

static Plan make_plan(const mi355_fa_params* p, int cus, bool allow_stage = true) {
  Plan pl{};
  const mi355_fa_variant v = variant_of(p);
  pl.pack = pick_pack(p, v);
  pl.num_n = ceil_div(p->seqlen_k, kBN);
  const int bh = p->b * p->h;
  int s_fixed = p->num_splits > 0 ? p->num_splits : env_num_splits();
  if (s_fixed > kMaxSplits) s_fixed = kMaxSplits;
  if (s_fixed > pl.num_n) s_fixed = pl.num_n;
  const int w_fixed = (v.waves == 4 || v.waves == 8) ? v.waves : 0;
  const PlanCost& cm = p->d == 64 ? kCostD64 : kCostD128;
  int max_s = pl.num_n / 4 > 1 ? pl.num_n / 4 : 1;
  if (max_s > kMaxSplits) max_s = kMaxSplits;
  float best = 0.f;
  pl.waves = 0;
  for (int w = 4; w <= 8; w += 4) {
    if (w_fixed && w != w_fixed) continue;
    for (int s = s_fixed > 0 ? s_fixed : 1; s <= (s_fixed > 0 ? s_fixed : max_s); ++s) {
      const float c = plan_cost(cm, bh, p->seqlen_q, pl.num_n, p->d, w, s, cus, pl.pack);
      if (pl.waves == 0 || c < best) { best = c; pl.waves = w; pl.splits = s; }
    }
  }
  if (pl.splits < 1) pl.splits = 1;
  const int s = pl.splits;
  pl.block_m = 32 * pl.waves;
  // Workgroup order. Each XCD runs a contiguous range of tile ids with its own
  // L2 (4 MiB, too small to keep a batch's K/V or mask between rounds), so
  // what one round of an XCD's workgroups fetches is what counts: the K/V of
  // the head groups it covers plus the mask rows of the m-blocks it covers.
  // m-blocks fastest covers few head groups and many m-blocks, heads fastest
  // the reverse; take the order whose round fetches fewer bytes. (MHA with
  // long Sq: m-blocks fastest; GQA, whose packed head groups share K/V, and
  // short Sq: heads fastest.)
  pl.head_major = order_head_major(p, pl, cus, v);
  pl.num_m = ceil_div(p->seqlen_q, pl.block_m / pl.pack);
  pl.n_per_split = (s > 1) ? ceil_div(pl.num_n, s) : pl.num_n;
  if (s > 1) {
    const size_t rows = (size_t)s * p->b * p->h * p->seqlen_q;
    pl.o_part_bytes = (rows * p->d * sizeof(uint16_t) + 255) & ~(size_t)255;
    pl.lse_bytes = (rows * sizeof(float) + 255) & ~(size_t)255;
    // one ticket word per row block (batch, head group, m-block)
    const size_t tickets = (size_t)p->b * (p->h / pl.pack) * pl.num_m;
    pl.ticket_bytes = (tickets * 8 + 255) & ~(size_t)255;
    // fused tail: two splits (the last one's combine reads two partials per
    // row); more splits keep the combine launch, whose work spreads over the
    // whole chip instead of falling on each row block's last split
    pl.fuse = s <= kFuseMaxSplits && pl.o_part_bytes < (1ull << 31) && pl.lse_bytes < (1ull << 31) &&
              v.fuse >= 0;
  }
  pl.loop = v.loop < 0 ? 0 : (v.loop >= 1 && v.loop <= 3 ? v.loop : 3);
  pl.live = v.live < 0 ? 0 : (v.live > 0 ? 1 : 2);
  // A mask whose rows are not 16-byte aligned goes through a pre-pass that
  // copies it to an aligned staged mask in the workspace (rows < Sq, columns
  // padded with -inf to a multiple of 8), so that every kernel takes its mask
  // tiles by LDS DMA, and writes the live-tile map that serves the live
  // ranges in place of each workgroup's scan. Variant stage = -1 (and callers
  // without room for the copy) keep the mask in place: the compiled kernel
  // then reads it through registers, with the map.
  {
    const bool mask_direct = ((uintptr_t)p->mask & 15) == 0 && (p->mask_batch_stride & 7) == 0 &&
                             (p->mask_row_stride & 7) == 0;
    // The map also serves 8-wave split launches of aligned masks, whose
    // workgroups would otherwise each scan their rows' dead mask: with the
    // heads and splits that share a row block, a window or causal mask reads
    // its dead part dozens of times ([2,16,16,1000,4096] window 122.8 -> 47.2
    // µs, top-left causal [2,16,4,1000,4096] 55.2 -> 37.0) while a dense mask
    // pays the pre-pass (78.5 -> 81.4). 4-wave deep launches (one workgroup
    // per CU, split-KV decode shapes such as cfg4) keep the scan: there the
    // pre-pass is pure latency on a dense mask (4.4 µs, cfg4 +6 %), however
    // many times a sparse one is re-read; Variant(live_map=1) forces the map.
    pl.live_map = (!mask_direct || v.live_map > 0 || (s > 1 && pl.waves == 8)) && pl.live != 0 &&
                  pl.num_n >= 4 && v.live_map >= 0;
    pl.map_row_bytes = ceil_div(pl.num_n, 8);
    pl.map_slices = ceil_div(p->seqlen_q, 16);
    pl.map_full_off = (int64_t)(((size_t)p->b * pl.map_slices * pl.map_row_bytes + 255) & ~(size_t)255);
    pl.map_bytes = pl.live_map ? (size_t)pl.map_full_off + (((size_t)p->b * pl.map_slices + 255) & ~(size_t)255)
                               : 0;
    pl.stage_rs = ceil_div(p->seqlen_k, 8) * 8;
    // Staged, the mask reaches the assembly loops and the LDS-DMA path of the
    // compiled kernel, which outrun the register path by more than the copy
    // costs: [4,16,16,2048,2047] random mask 150 against 178 µs, top-left
    // causal 139 against 157; cfg5's shape (8 waves, 2 splits, the ping-pong
    // loop with the map) window 44.2 against 46.5, 10 % random 85.3 against
    // 93.4 (same sessions, hot).
    pl.staged = !mask_direct && allow_stage && v.stage >= 0 && p->seqlen_k >= 8 &&
                (uint64_t)p->seqlen_q * pl.stage_rs * 2 < (1ull << 31);
    pl.stage_bytes = pl.staged ? (((size_t)p->b * p->seqlen_q * pl.stage_rs * 2 + 255) & ~(size_t)255) : 0;
  }
  pl.ws_bytes = pl.o_part_bytes + pl.lse_bytes + pl.ticket_bytes + pl.map_bytes + pl.stage_bytes;
  // A 4-wave grid that puts at most one workgroup on each CU takes a third K/V
  // stage (112 KiB of LDS at d = 128: one workgroup per CU; cfg4 cold -7 %).
  {
    const int64_t wgs = (int64_t)p->b * (p->h / pl.pack) * pl.num_m * s;
    pl.deep = (pl.waves == 4 && wgs <= cus && v.deep >= 0) ? 1 : 0;
  }
  pl.mask_mfma_off = v.mask_mfma < 0 ? 1 : 0;
  // One m-block per head group and every q-head of a KV head in the same
  // workgroup: each K/V tile is read by exactly one workgroup of the launch
  // (split-KV decode shapes such as Sq 128 x Sk 32k), a stream with no reuse
  // for the caches to keep. Loaded non-temporally, its cold read runs at the
  // rate a plain streaming read reaches with that hint (7.2 against 6.5 TB/s
  // on MI355X); a back-to-back repeat of the same call that could have found
  // part of it in the 256 MiB last-level cache loses that.
  pl.kv_nt = v.stream < 0 ? 0 : (v.stream > 0 ? 1 : (pl.num_m == 1 && pl.pack == p->h / p->h_k));
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
    // 16-byte vector access to q/k/v/o rows (O leaves in 16-byte row chunks)
    const uintptr_t al = (uintptr_t)p->q | (uintptr_t)p->o | (uintptr_t)p->k | (uintptr_t)p->v;
    const int64_t st = p->q_batch_stride | p->q_head_stride | p->q_row_stride | p->k_batch_stride |
                       p->k_head_stride | p->k_row_stride | p->v_batch_stride | p->v_head_stride |
                       p->v_row_stride | p->o_batch_stride | p->o_head_stride | p->o_row_stride;
    if ((al & 15) || (st & 7)) {
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

template <int D, bool BF16, bool SPLIT, int WAVES, bool DEEP>
static hipError_t launch_main(const KParams& kp, hipStream_t st) {
  constexpr int NST = WAVES == 8 ? MI355_FA_STAGES8 : (DEEP && MI355_FA_STAGES4 < 3 ? 3 : MI355_FA_STAGES4);
  const size_t dyn = DEEP ? (size_t)(NST - 2) * (Geo<D, WAVES>::kKElems + Geo<D, WAVES>::kVElems) * 2 : 0;
  if (kp.mask_direct && WAVES == 4 && DEEP && kp.live_map)
    hipLaunchKernelGGL((fa_fwd_kernel<D, BF16, SPLIT, true, WAVES, DEEP, true>), dim3(kp.total),
                       dim3(64 * WAVES), dyn, st, kp);
  else if (kp.mask_direct)
    hipLaunchKernelGGL((fa_fwd_kernel<D, BF16, SPLIT, true, WAVES, DEEP>), dim3(kp.total),
                       dim3(64 * WAVES), dyn, st, kp);
  else
    hipLaunchKernelGGL((fa_fwd_kernel<D, BF16, SPLIT, false, WAVES, DEEP>), dim3(kp.total),
                       dim3(64 * WAVES), dyn, st, kp);
  return hipGetLastError();
}

// A 48-bit launch tag, never 0, distinct for every launch of the process
// (splitmix64 of a per-process random seed plus a launch counter): a ticket
// word left by an earlier launch in reused workspace memory carries another
// tag, so the first split of this launch restarts its count.
static unsigned long long next_launch_tag() {
  static std::atomic<unsigned long long> ctr{0};
  static const unsigned long long seed = [] {
    std::random_device rd;
    return ((unsigned long long)rd() << 32) ^ rd() ^
           (unsigned long long)std::chrono::steady_clock::now().time_since_epoch().count();
  }();
  unsigned long long z = seed + 0x9e3779b97f4a7c15ull * (ctr.fetch_add(1) + 1);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  z ^= z >> 31;
  z &= (1ull << 48) - 1;
  return z ? z : 1ull;
}

// Whether a launch runs one of the generated-assembly loops (d = 128, 8-wave
// plans, 16-byte aligned mask rows) rather than the compiled kernel.
template <int D, bool BF16>
static bool runs_asm_loop(const KParams& kp, const Plan& pl) {
  // bf16 adds the mask on the matrix core, which needs bf16(1/scale) > 1.0078
  // (-max_bf16 · (1/scale) must overflow to -inf): scale < 0.99
  return D == 128 && pl.waves == 8 && kp.mask_direct && pl.loop && (!BF16 || kp.scale < 0.99f);
}

template <int D, bool BF16, bool SPLIT>
static hipError_t launch_variant(const KParams& kp, const Plan& pl, hipStream_t st) {
  if constexpr (D == 128) {
    if (runs_asm_loop<D, BF16>(kp, pl)) {
      if (pl.loop == 3 && BF16)
        if (kp.live_map)
          hipLaunchKernelGGL((fa_fwd_kernel_pp<SPLIT, true>), dim3(kp.total), dim3(512), 0, st, kp);
        else
          hipLaunchKernelGGL((fa_fwd_kernel_pp<SPLIT, false>), dim3(kp.total), dim3(512), 0, st, kp);
      else if (pl.loop == 2)
        hipLaunchKernelGGL((fa_fwd_kernel_asm<2, BF16, SPLIT>), dim3(kp.total), dim3(256), 0, st, kp);
      else
        hipLaunchKernelGGL((fa_fwd_kernel_asm<1, BF16, SPLIT>), dim3(kp.total), dim3(512), 0, st, kp);
      return hipGetLastError();
    }
  }
  if (pl.waves == 8) return launch_main<D, BF16, SPLIT, 8, false>(kp, st);
  return pl.deep ? launch_main<D, BF16, SPLIT, 4, true>(kp, st) : launch_main<D, BF16, SPLIT, 4, false>(kp, st);
}

template <int D, bool BF16>
static hipError_t launch(const KParams& kp_in, const CParams& cp, const Plan& pl, hipStream_t st) {
  KParams kp = kp_in;
  const int lm = pl.live;
  kp.live = pl.num_n >= 4 && (lm == 1 || (lm == 2 && (pl.splits > 1 || !runs_asm_loop<D, BF16>(kp, pl))));
  // the kernels that read the map: the compiled kernel and the ping-pong loop
  // (the 32- and 64-row loops scan)
  const bool reads_map = !runs_asm_loop<D, BF16>(kp, pl) || (D == 128 && BF16 && pl.loop == 3);
  const bool want_map = kp.live && kp.live_map_out && reads_map;
  if (kp.stage_out || want_map) {
    KParams km = kp;
    if (!want_map) km.live_map_out = nullptr;
    hipLaunchKernelGGL((mask_stage_kernel<BF16>), dim3((unsigned)(kp.b * kp.map_slices * kp.map_row_bytes)),
                       dim3(256), 0, st, km);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  kp.live_map = want_map ? kp.live_map_out : nullptr;
  if (pl.splits == 1) return launch_variant<D, BF16, false>(kp, pl, st);
  // the fused tail is in the compiled kernel only (the assembly loops keep no
  // registers for it): their split launches keep the combine launch
  KParams kf = kp;
  kf.fuse = kp.fuse && !runs_asm_loop<D, BF16>(kp, pl);
  hipError_t e = launch_variant<D, BF16, true>(kf, pl, st);
  if (e != hipSuccess || kf.fuse) return e;
  // 256-thread workgroups while they still number >= 1024, else one wave each.
  constexpr int kRows256 = 256 / (D / 8), kRows64 = 64 / (D / 8);
  if ((cp.rows + kRows256 - 1) / kRows256 >= 1024) {
    hipLaunchKernelGGL((fa_combine_kernel<D, BF16, 256>),
                       dim3((unsigned)((cp.rows + kRows256 - 1) / kRows256)), dim3(256), 0, st, cp);
  } else {
    hipLaunchKernelGGL((fa_combine_kernel<D, BF16, 64>),
                       dim3((unsigned)((cp.rows + kRows64 - 1) / kRows64)), dim3(64), 0, st, cp);
  }
  return hipGetLastError();
}

}  // namespace mi355fa

using namespace mi355fa;

extern "C" {

int mi355_fa_abi_version(void) { return MI355_FA_ABI_VERSION; }

const char* mi355_fa_build_info(void) {
  return "mi355_fa gfx950 BM=128/256 BN=64 32-rows/wave mfma32x32x16 lds-dma tr-reads splitkv+combine";
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

}  // extern "C"

// The launch behind both entry points; allow_stage false plans without the
// staged mask (mi355_fa_fwd_noalloc when the copy would not fit its scratch).
static int fwd_impl(const mi355_fa_params* p, void* stream, char* err, size_t errlen, bool allow_stage) {
  int rc = validate(p, err, errlen);
  if (rc) return rc;
  if (p->b == 0 || p->h == 0 || p->seqlen_q == 0) return MI355_FA_OK;
  const DeviceInfo dev = device_info();
  if (!dev.gfx950) {
    set_err(err, errlen, "mi355_fa: current HIP device is not gfx950 (MI355X)");
    return MI355_FA_EDEVICE;
  }
  const Plan pl = make_plan(p, dev.cus, allow_stage);
  const int64_t total = (int64_t)p->b * (p->h / pl.pack) * pl.num_m * pl.splits;
  if (total >= (1LL << 24)) {
    set_err(err, errlen, "problem too large: %lld workgroups", (long long)total);
    return MI355_FA_EINVAL;
  }
  // Buffer offsets are 32-bit: every per-head / per-batch byte range the kernel
  // addresses (including the rounded-up last row tile) must stay below 2^32.
  {
    const uint64_t rows_q = (uint64_t)pl.num_m * (pl.block_m / pl.pack), rows_k = (uint64_t)pl.num_n * kBN;
    const uint64_t lim = 0xffffffffull - 4096;
    const uint64_t need[] = {
        rows_q * (uint64_t)p->q_row_stride * 2, rows_q * (uint64_t)p->o_row_stride * 2,
        rows_k * (uint64_t)p->k_row_stride * 2, rows_k * (uint64_t)p->v_row_stride * 2,
        (rows_q * (uint64_t)p->mask_row_stride + rows_k) * 2,
        (uint64_t)p->mask_seqlen_q * (uint64_t)p->mask_row_stride * 2};
    for (uint64_t n : need) {
      if (n > lim) {
        set_err(err, errlen, "problem too large: a per-head or per-batch tensor slice exceeds 4 GiB");
        return MI355_FA_EINVAL;
      }
    }
  }
  const bool split = pl.splits > 1;
  if (pl.ws_bytes && (!p->workspace || p->workspace_bytes < pl.ws_bytes)) {
    set_err(err, errlen, "%s needs %zu workspace bytes, got %zu",
            split ? "split-KV" : (pl.staged ? "the staged mask" : "the live-tile map"), pl.ws_bytes,
            p->workspace_bytes);
    return MI355_FA_EWORKSPACE;
  }

  KParams kp{};
  kp.q = (const uint16_t*)p->q;
  kp.k = (const uint16_t*)p->k;
  kp.v = (const uint16_t*)p->v;
  kp.mask = (const uint16_t*)p->mask;
  kp.o = (uint16_t*)p->o;
  kp.q_bs = p->q_batch_stride; kp.q_hs = p->q_head_stride; kp.q_rs = (int)p->q_row_stride;
  kp.k_bs = p->k_batch_stride; kp.k_hs = p->k_head_stride; kp.k_rs = (int)p->k_row_stride;
  kp.v_bs = p->v_batch_stride; kp.v_hs = p->v_head_stride; kp.v_rs = (int)p->v_row_stride;
  kp.o_bs = p->o_batch_stride; kp.o_hs = p->o_head_stride; kp.o_rs = (int)p->o_row_stride;
  kp.m_bs = p->mask_batch_stride; kp.m_rs = (int)p->mask_row_stride;
  kp.b = p->b; kp.h = p->h; kp.ratio = p->h / p->h_k; kp.pack = pl.pack;
  kp.sq = p->seqlen_q; kp.sk = p->seqlen_k; kp.msq = p->mask_seqlen_q;
  kp.num_m = pl.num_m; kp.num_n = pl.num_n;
  kp.num_splits = pl.splits; kp.n_per_split = pl.n_per_split;
  kp.total = (int)total;
  kp.scale = p->scale_softmax;
  kp.mask_mfma = (p->dtype == MI355_FA_BF16 && p->scale_softmax < 0.99f && !pl.mask_mfma_off) ? 1 : 0;
  kp.kv_nt = pl.kv_nt;
  {
    const float c2 = p->scale_softmax * kLog2e, slack = kRescaleSlack / p->scale_softmax;
    memcpy(&kp.c2_bits, &c2, 4);
    memcpy(&kp.slack_bits, &slack, 4);
  }
  kp.head_major = pl.head_major;
  kp.mask_direct = (((uintptr_t)p->mask & 15) == 0 && (p->mask_batch_stride & 7) == 0 &&
                    (p->mask_row_stride & 7) == 0) ? 1 : 0;

  // the live-tile map and the staged mask (workspace after the split
  // partials and tickets)
  kp.msrc = kp.mask; kp.msrc_bs = kp.m_bs; kp.msrc_rs = kp.m_rs; kp.msrc_q = kp.msq;
  kp.map_row_bytes = pl.map_row_bytes;
  kp.map_slices = pl.map_slices;
  kp.map_full_off = pl.map_full_off;
  if (pl.live_map)
    kp.live_map_out = (uint8_t*)p->workspace + pl.o_part_bytes + pl.lse_bytes + pl.ticket_bytes;
  if (pl.staged) {
    kp.stage_out = (uint16_t*)((char*)p->workspace + pl.o_part_bytes + pl.lse_bytes + pl.ticket_bytes +
                               pl.map_bytes);
    kp.stage_rs = pl.stage_rs;
    kp.mask = kp.stage_out;
    kp.m_rs = pl.stage_rs;
    kp.m_bs = (int64_t)p->seqlen_q * pl.stage_rs;
    kp.msq = p->seqlen_q;
    kp.mask_direct = 1;
  }

  CParams cp{};
  if (split) {
    kp.o_part = (uint16_t*)p->workspace;
    kp.lse_part = (float*)((char*)p->workspace + pl.o_part_bytes);
    kp.tickets = (unsigned long long*)((char*)p->workspace + pl.o_part_bytes + pl.lse_bytes);
    kp.fuse = pl.fuse;
    kp.tag = pl.fuse ? next_launch_tag() : 0ull;
    kp.part_bytes = (uint32_t)std::min<size_t>(pl.o_part_bytes, 0xffffffffu);
    kp.lse_bytes = (uint32_t)std::min<size_t>(pl.lse_bytes, 0xffffffffu);
    cp.o_part = kp.o_part;
    cp.lse_part = kp.lse_part;
    cp.o = kp.o;
    cp.o_bs = kp.o_bs; cp.o_hs = kp.o_hs; cp.o_rs = kp.o_rs;
    cp.b = p->b; cp.h = p->h; cp.sq = p->seqlen_q; cp.num_splits = pl.splits;
    cp.rows = (int64_t)p->b * p->h * p->seqlen_q;
    cp.part_bytes = pl.o_part_bytes < (1ull << 31) ? (uint32_t)pl.o_part_bytes : 0u;
  }

  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  const bool bf16 = p->dtype == MI355_FA_BF16;
  if (p->d == 128)
    e = bf16 ? launch<128, true>(kp, cp, pl, st) : launch<128, false>(kp, cp, pl, st);
  else
    e = bf16 ? launch<64, true>(kp, cp, pl, st) : launch<64, false>(kp, cp, pl, st);
  if (e != hipSuccess) {
    set_err(err, errlen, "mi355_fa launch failed: %s", hipGetErrorString(e));
    return MI355_FA_ELAUNCH;
  }
  return MI355_FA_OK;
}

extern "C" int mi355_fa_fwd(const mi355_fa_params* p, void* stream, char* err, size_t errlen) {
  return fwd_impl(p, stream, err, errlen, true);
}

// ── entry point that allocates nothing ───────────────────────────────────────
// mi355_fa_fwd_noalloc keeps the split-KV partials in this file-scope device
// array instead of a caller workspace: one copy per GPU, resident until the
// process ends. Host code never passes the array's name to a kernel (on the
// host it is only a stand-in symbol); it uses the device address that
// hipGetSymbolAddress returns for the current device, looked up once per
// device on that device's first call. Partials are fully written before they
// are read, so nothing needs clearing between calls; calls that overlap on one
// GPU share the array and race.
static __device__ __align__(256) unsigned char scratch[MI355_FA_NOALLOC_SCRATCH_BYTES];

static void* g_scratch_ptr[64];
static std::mutex g_scratch_mu;

static int scratch_of_current_device(void** out, char* err, size_t errlen) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    set_err(err, errlen, "mi355_fa: no current HIP device (%s)", hipGetErrorString(e));
    return MI355_FA_EDEVICE;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      (void)hipGetLastError();
      set_err(err, errlen, "mi355_fa: scratch address lookup failed on device %d: %s", dev,
              hipGetErrorString(e));
      return MI355_FA_ELAUNCH;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MI355_FA_OK;
}

extern "C" int mi355_fa_fwd_noalloc(const mi355_fa_params* p, void* stream, char* err, size_t errlen) {
  int rc = validate(p, err, errlen);
  if (rc) return rc;
  if (p->b == 0 || p->h == 0 || p->seqlen_q == 0) return MI355_FA_OK;
  // the staged mask when it fits the scratch, else the mask read in place
  size_t need = mi355_fa_workspace_bytes(p);
  bool allow_stage = true;
  if (need > MI355_FA_NOALLOC_SCRATCH_BYTES) {
    allow_stage = false;
    need = make_plan(p, device_info().cus, false).ws_bytes;
  }
  if (need > MI355_FA_NOALLOC_SCRATCH_BYTES) {
    set_err(err, errlen,
            "split-KV needs %zu bytes of scratch; mi355_fa_fwd_noalloc holds at most %zu "
            "(use mi355_fa_fwd with a workspace, or fewer splits)",
            need, (size_t)MI355_FA_NOALLOC_SCRATCH_BYTES);
    return MI355_FA_EWORKSPACE;
  }
  mi355_fa_params q = *p;
  q.workspace = nullptr;
  q.workspace_bytes = 0;
  if (need > 0) {
    rc = scratch_of_current_device(&q.workspace, err, errlen);
    if (rc) return rc;
    q.workspace_bytes = MI355_FA_NOALLOC_SCRATCH_BYTES;
  }
  return fwd_impl(&q, stream, err, errlen, allow_stage);
}
