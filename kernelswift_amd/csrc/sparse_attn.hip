// Sparse attention over gathered top-k KV rows with an attention sink (gfx950).
//
// Semantics: sparse_attn_ref (baseline/sparse_attention.py:5-42); replaces the reference's kvT transpose +
// dense-N megakernel (optimized/sparse_attention/op_kernel/fused_sparse_attn_basic_kernel.asc:535-648,
// transpose_kv_kernel.asc:35-63), which only handled N = 32 keys, with a real gather.
//
// Work item = (query (b, m), key range).  A group of GW waves (16 heads each) owns one item; a workgroup
// holds GROUPS groups (as many as 8 waves and the LDS budget allow).  The group walks its key range in
// chunks of 32 keys.  Each chunk's kv rows are gathered straight into LDS with global_load_lds_dwordx4
// (no VGPR round trip): a DMA instruction writes 64 consecutive 16-byte slots, one per lane, and the lane
// chooses which (key, unit) it fetches, so the buffer holds the rows in a swizzled row-major layout
// (unit u of key k in slot k*UPR + (u ^ swz(k))) that keeps both read patterns below free of bank
// conflicts.  Two buffers: chunk c + 1 is in flight while chunk c is computed; the row indices are fetched
// one chunk further ahead; one barrier per chunk.
//   QK^T   S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (M = 16 keys, N = 16 heads), q rows as B-fragments
//          in VGPRs; lane (head = l%16, g = l/16) receives keys 16t + 4g + r (t = 0, 1; r = 0..3).
//   softmax online in base 2 with a lazily updated reference max (rescale only when a chunk's max exceeds
//          it by more than 2^8), invalid keys -> 0.
//   PV     O = P V (M = 16 heads, N = 16 dv columns, K = 32 keys).  A lane's 8 probabilities are its
//          A-fragment as they are; the matching V fragment (keys 4g..4g+3 and 16+4g..16+4g+3 of one column)
//          comes from the same buffer with two ds_read_b64_tr_b16 transpose reads, so V is neither copied
//          nor transposed.
// One range per query finalises in place (sink added, bf16 store); otherwise partial (O, max, sum) go to
// the workspace and a combine kernel merges the ranges with the sink (one wave per output row).
// MLA-shaped heads (Dqk 576, Dv 512, H a multiple of 32) use sparse_attn_mla_kernel below: 32 heads per
// wave, one wave per SIMD, O accumulated in AGPRs.
#include "common.h"

#include <array>
#include <mutex>

namespace ks {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kKC = 32;               // keys per chunk
constexpr int kLdsBudget = 160 * 1024 - 1024;
constexpr int kTargetWaves = 2048;    // waves in flight the split heuristic aims for
constexpr int kMinChunks = 4;         // at least this many chunks per work item
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleTau = 8.f;    // lazy rescale threshold (log2 units): probabilities stay <= 2^8

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                  0, 0, 0);
}

// Two fp32 -> packed bf16 (RNE), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// 2^x with the hardware transcendental (v_exp_f32); softmax weights need no denormal results.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ds_read_b64_tr_b16: within each 16-lane row, lane i receives element i%4 of the 8-byte rows addressed by
// lanes 4e + i/4 (e = 0..3), i.e. a 4 x 4 block transpose of 16-bit elements across lane quads.
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t *p) {
  typedef __attribute__((address_space(3))) short4_t lds_short4_t;
  const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t *)(const_cast<uint16_t *>(p)));
  return __builtin_bit_cast(uint2, v);
}

// A wave-uniform pointer moved to SGPRs (the compiler cannot prove uniformity of values derived from the
// wave index).  The result is typed as a global-memory pointer: rebuilt from an integer, a generic pointer
// would make its loads flat loads, which also count in lgkmcnt, so every wait for an LDS read would then
// wait for them too.
template <typename T>
using global_ptr = __attribute__((address_space(1))) T *;
template <typename T>
__device__ __forceinline__ global_ptr<T> uniform_ptr(T *p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<global_ptr<T>>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Reductions over the four 16-lane rows of the wave (lanes l, l^16, l^32, l^48), result in every lane:
// v_permlane16_swap exchanges rows 1/3 of its first operand with rows 0/2 of its second, so with the value
// in both operands each lane holds its row pair's two values; v_permlane32_swap does the same across the
// wave halves.  Inline assembly (the builtin form was miscompiled into v op v when both operands carry the
// same value); the NOPs cover the VALU-write -> permlane-read hazard.
__device__ __forceinline__ void swap16(float &a, float &b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float &a, float &b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float rows_max(float v) {
  float a = v, b = v;
  swap16(a, b);
  float c = fmaxf(a, b), d = c;
  swap32(c, d);
  return fmaxf(c, d);
}
__device__ __forceinline__ float rows_sum(float v) {
  float a = v, b = v;
  swap16(a, b);
  float c = a + b, d = c;
  swap32(c, d);
  return c + d;
}

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int DQK, int DV, int GW>
struct SaShape {
  static constexpr int UPR = DQK / 8;  // 16-byte units per row
  static constexpr int NTG = 64 * GW;  // threads per group
  static constexpr int UNITS = kKC * UPR;
  static constexpr int TI = UNITS / 64;          // DMA instructions per chunk (64 slots each)
  static constexpr int NJ = (TI + GW - 1) / GW;  // ... per wave
  static constexpr int BUF = UNITS * 8;          // bf16 elements per chunk buffer
  // q fragments (one uint4 per lane and k-step): the first QREG k-steps stay in VGPRs, the rest in LDS
  // (wide heads: 16 heads x 576 dims of q plus 16 x 512 fp32 accumulators would not fit 256 VGPRs)
  static constexpr int QJ = DQK / 32;
  static constexpr int QREG = DQK > 256 ? QJ / 2 : QJ;
  static constexpr int QL = QJ - QREG;
  static constexpr int GROUP_BYTES = 2 * BUF * 2 + GW * (QL > 0 ? QL : 0) * 64 * 16;
  static constexpr int FIT = kLdsBudget / GROUP_BYTES;
  static constexpr int GROUPS = (8 / GW) < FIT ? (8 / GW) : FIT;
  static constexpr int THREADS = GROUPS * NTG;
  static_assert(GROUPS >= 1, "one group must fit in LDS");
  static_assert(UNITS % 64 == 0 && UPR % 8 == 0, "chunk must be whole DMA instructions");
  // Slot of unit u of key k.  Rows of 16 units start on bank 0: XOR with 2(k & 7) spreads 8 keys over the
  // 8 odd/even unit pairs; rows of 72 units alternate between bank halves: XOR with k & 7 suffices.
  static constexpr int SW = UPR % 16 == 0 ? 16 : 8;  // the XOR touches unit bits below SW
  __device__ static __forceinline__ int swz(int k) { return UPR % 16 == 0 ? (k & 7) << 1 : (k & 7); }
  // slot of unit u = u_hi + u_lo with u_hi a compile-time multiple of SW and 0 <= u_lo < SW: written so
  // that u_hi folds into the LDS instruction's immediate offset
  __device__ static __forceinline__ int slot(int k, int u_hi, int u_lo) { return k * UPR + u_hi + (u_lo ^ swz(k)); }
};

inline int waves_per_group(int64_t H) {
  const int64_t w = (H + 15) / 16;
  return w <= 1 ? 1 : w <= 2 ? 2 : w <= 4 ? 4 : 8;
}

// Key ranges per query: enough work items for ~kTargetWaves waves, at least kMinChunks chunks each.
inline int choose_splits(int64_t B, int64_t M, int64_t H, int64_t K) {
  const int64_t waves_base = B * M * waves_per_group(H);
  const int64_t chunks = (K + kKC - 1) / kKC;
  int64_t ns = (kTargetWaves + waves_base - 1) / (waves_base > 0 ? waves_base : 1);
  const int64_t cap = chunks / kMinChunks > 1 ? chunks / kMinChunks : 1;
  if (ns > cap) ns = cap;
  if (ns > 64) ns = 64;
  if (ns < 1) ns = 1;
  return static_cast<int>(ns);
}

struct SaSplit {
  int ns;   // ranges actually used
  int kr;   // keys per range (multiple of kKC)
};

inline SaSplit split_plan(int64_t B, int64_t M, int64_t H, int64_t K) {
  const int ns0 = choose_splits(B, M, H, K);
  const int64_t chunks = (K + kKC - 1) / kKC;
  const int64_t kr = ((chunks + ns0 - 1) / ns0) * kKC;
  return SaSplit{static_cast<int>((K + kr - 1) / kr), static_cast<int>(kr)};
}

template <int DQK, int DV, int GW>
__global__ __launch_bounds__((SaShape<DQK, DV, GW>::THREADS)) void sparse_attn_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ kv, const float *__restrict__ sink,
    const int32_t *__restrict__ idx, uint16_t *__restrict__ out, uint16_t *__restrict__ part_o,
    float *__restrict__ part_ml, int64_t n_items, int64_t M, int H, int64_t N, int64_t K, int NS, int KR,
    float scale_log2) {
  using Sh = SaShape<DQK, DV, GW>;
  constexpr int QJ = Sh::QJ, QREG = Sh::QREG, QL = Sh::QL;  // k-steps of the QK MFMA
  constexpr int CT = DV / 16;   // dv column tiles
  constexpr int UPR = Sh::UPR, NJ = Sh::NJ;
  __shared__ __attribute__((aligned(16))) uint16_t kb[Sh::GROUPS][2][Sh::BUF];
  __shared__ __attribute__((aligned(16))) uint4 qs[Sh::GROUPS][GW][QL > 0 ? QL : 1][64];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps item / row math scalar
  const int grp = wave / GW, gw = wave % GW;
  const int l16 = lane & 15, g = lane >> 4;
  // Workgroups are dealt to the 8 XCDs round-robin (block id mod 8); consecutive logical workgroups (the
  // ranges of one query, which share its q rows) are placed on one XCD so that they share its L2.
  const int64_t nblk = gridDim.x;
  const int64_t wg = (nblk % 8 == 0) ? (blockIdx.x % 8) * (nblk / 8) + blockIdx.x / 8 : blockIdx.x;
  const int64_t item = wg * Sh::GROUPS + grp;
  const bool item_ok = item < n_items;
  const int64_t qm = item_ok ? item / NS : 0;
  const int split = item_ok ? static_cast<int>(item % NS) : 0;
  const int64_t b = qm / M;
  const int head = gw * 16 + l16;
  const bool head_ok = item_ok && head < H;
  const int k_begin = split * KR;  // K < 2^31 (host-checked): key positions fit int32
  const int k_end = item_ok ? (k_begin + KR < K ? k_begin + KR : static_cast<int>(K)) : k_begin;
  const global_ptr<const int32_t> irow = uniform_ptr(idx + qm * K);
  const global_ptr<const uint16_t> kvb = uniform_ptr(kv + b * N * DQK);
  const int nch = (KR + kKC - 1) / kKC;  // the same for every group of the workgroup

  // DMA slot 64 (gw + GW i) + lane of a chunk holds unit u_i of key key_i (fixed per lane).
  int key_i[NJ], uoff_i[NJ];
#pragma unroll
  for (int i = 0; i < NJ; ++i) {
    const int sl = 64 * (gw + GW * i) + lane;
    key_i[i] = sl / UPR;
    uoff_i[i] = ((sl % UPR) ^ Sh::swz(key_i[i])) * 16;  // the XOR is an involution
  }
  const uint32_t kb_lds = __builtin_amdgcn_readfirstlane(lds_addr(&kb[grp][0][0]));
  const int n32 = static_cast<int>(N), k32 = static_cast<int>(K);
  // Raw indices of chunk c: for each DMA slot i, and for key (lane & 31) (validity mask).  Loaded without
  // a branch and validated only where they are used one chunk later, so no wait is placed behind the loads.
  auto raw_idx = [&](int c, int key) -> int32_t {
    const int t = k_begin + c * kKC + key;
    return irow[t < k32 ? t : k32 - 1];
  };
  // bit k: key k of chunk c is valid (inside the range, index in [0, N)); wave-uniform
  auto valid_mask = [&](int c, int32_t vraw) -> uint32_t {
    const bool ok = k_begin + c * kKC + (lane & 31) < k_end && vraw >= 0 && vraw < n32;
    return static_cast<uint32_t>(__builtin_amdgcn_ballot_w64(ok));
  };
  // gather chunk c's rows into buffer `buf` (invalid keys read row 0: finite data, masked by `vm`)
  auto gather = [&](const int32_t(&raw)[NJ], uint32_t vm, int buf) {
#pragma unroll
    for (int i = 0; i < NJ; ++i) {
      const int jj = gw + GW * i;
      if (jj < Sh::TI) {
        const bool ok = (vm >> key_i[i]) & 1u;
        const uint32_t voff = static_cast<uint32_t>(ok ? raw[i] : 0) * (DQK * 2) + uoff_i[i];
        dma16((const void *)kvb, voff, kb_lds + (buf * Sh::BUF + 64 * jj * 8) * 2);
      }
    }
  };

  // chunk 0's indices first, then the q B-fragments (Q[head][32j + 8g .. +7]): the first gather waits for the
  // indices alone and is in flight with the q loads
  int32_t nraw[NJ];
#pragma unroll
  for (int i = 0; i < NJ; ++i) nraw[i] = raw_idx(0, key_i[i]);
  int32_t nvraw = raw_idx(0, lane & 31);
  uint4 qf[QREG];
#pragma unroll
  for (int j = 0; j < QJ; ++j) {
    const uint4 v = head_ok ? *reinterpret_cast<const uint4 *>(q + (qm * H + head) * DQK + 32 * j + 8 * g)
                            : make_uint4(0, 0, 0, 0);
    if (j < QREG) qf[j < QREG ? j : 0] = v;
    else qs[grp][gw][j - QREG][lane] = v;
  }
  uint32_t vm_cur = valid_mask(0, nvraw);
  gather(nraw, vm_cur, 0);
  const int c1 = nch > 1 ? 1 : 0;
#pragma unroll
  for (int i = 0; i < NJ; ++i) nraw[i] = raw_idx(c1, key_i[i]);
  nvraw = raw_idx(c1, lane & 31);
  wait_dma();
  __syncthreads();  // also publishes the q fragments kept in LDS

  // Per-lane LDS element offsets of the swizzled reads, one per distinct low-unit pattern; the high unit
  // bits add compile-time offsets.  QK: key 16t + l16, unit 4j + g.  PV (transpose reads): keys
  // 4g + (l16 >> 2) (+16), unit 2cc + ((l16 & 3) >> 1), 8-byte half l16 & 1.
  int qk_off[2][Sh::SW / 4], pv_off[2][Sh::SW / 2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int p = 0; p < Sh::SW / 4; ++p) qk_off[t][p] = Sh::slot(16 * t + l16, 0, 4 * p + g) * 8;
    const int kv_key = 4 * g + (l16 >> 2) + 16 * t;
#pragma unroll
    for (int p = 0; p < Sh::SW / 2; ++p)
      pv_off[t][p] = Sh::slot(kv_key, 0, 2 * p + ((l16 & 3) >> 1)) * 8 + 4 * (l16 & 1);
  }

  float m_ref = -INFINITY, l_run = 0.f;  // per head (lane l16), replicated over g
  f32x4_t o[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c) o[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int c = 0; c < nch; ++c) {
    const int buf = c & 1;
    uint32_t vm_next = 0;
    if (c + 1 < nch) {  // chunk c + 1 into the other buffer while this one is computed
      vm_next = valid_mask(c + 1, nvraw);
      gather(nraw, vm_next, buf ^ 1);
      const int c2 = c + 2 < nch ? c + 2 : c + 1;
#pragma unroll
      for (int i = 0; i < NJ; ++i) nraw[i] = raw_idx(c2, key_i[i]);
      nvraw = raw_idx(c2, lane & 31);
    }
    const uint16_t *kbp = kb[grp][buf];
    // ---- S^T = K Q^T for the chunk's two 16-key tiles
    f32x4_t st[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      st[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < QJ; ++j) {
        constexpr int kPat = Sh::SW / 4;  // distinct (4j mod SW) patterns
        const uint16_t *a = kbp + qk_off[t][j % kPat] + ((4 * j) & ~(Sh::SW - 1)) * 8;
        st[t] = mfma16(*reinterpret_cast<const uint4 *>(a),
                       j < QREG ? qf[j < QREG ? j : 0] : qs[grp][gw][j < QREG ? 0 : j - QREG][lane], st[t]);
      }
    }
    // ---- online softmax (lane: head l16, keys 16t + 4g + r)
    const uint32_t vbits = vm_cur >> (4 * g);  // bit 16t + r: key 16t + 4g + r
    float sc[8];
    float cmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = (vbits >> (16 * t + r)) & 1u;
        const float sv = ok ? st[t][r] * scale_log2 : -INFINITY;
        sc[4 * t + r] = sv;
        cmax = fmaxf(cmax, sv);
      }
    cmax = rows_max(cmax);
    const bool need = cmax > m_ref + kRescaleTau;  // false for cmax = -inf; true for a first valid chunk
    if (__builtin_amdgcn_ballot_w64(need) != 0ull) {
      const float m_new = need ? cmax : m_ref;
      const float alpha = need ? (m_ref == -INFINITY ? 0.f : fast_exp2(m_ref - m_new)) : 1.f;
      l_run *= alpha;
      m_ref = m_new;
      // O rows are heads 4g + r; their alpha lives in lane 4g + r
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float ar = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
        for (int cc = 0; cc < CT; ++cc) o[cc][r] *= ar;
      }
    }
    float p[8], csum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = sc[i] == -INFINITY ? 0.f : fast_exp2(sc[i] - m_ref);
      csum += p[i];
    }
    l_run += rows_sum(csum);
    // ---- O += P V: V fragment of keys 16h + 4g + (l16 >> 2), dv columns 16cc + 4(l16 & 3) .. +3
    const uint4 pa = make_uint4(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                                pack_bf16x2(p[6], p[7]));
#pragma unroll
    for (int cc = 0; cc < CT; ++cc) {
      constexpr int kPat = Sh::SW / 2;  // distinct (2cc mod SW) patterns
      const int hi = ((2 * cc) & ~(Sh::SW - 1)) * 8;
      const uint2 b0 = lds_read_tr16(kbp + pv_off[0][cc % kPat] + hi);
      const uint2 b1 = lds_read_tr16(kbp + pv_off[1][cc % kPat] + hi);
      o[cc] = mfma16(pa, make_uint4(b0.x, b0.y, b1.x, b1.y), o[cc]);
    }
    // this wave's part of chunk c + 1 has landed (the DMA counts as a vector-memory load); with several
    // waves per group, a barrier then publishes everyone's part and releases buffer `buf` for refilling.
    // A one-wave group needs no barrier: its own reads of `buf` completed before the MFMAs that used them.
    wait_dma();
    if constexpr (GW > 1) __syncthreads();
    vm_cur = vm_next;
  }

  // Merge of the GROUPS ranges of one query held by this workgroup (one-wave groups): each wave leaves its
  // (max, sum) per head and its O in LDS (the chunk buffers are free now); the workgroup then combines
  // them per (head, column) and writes one partial range (or the output, when it covers the query).
  auto merge_groups = [&](const f32x4_t(&oo)[CT], float mr, float lr) {
    static_assert(Sh::GROUPS * 16 * DV * 4 + Sh::GROUPS * 32 * 4 <= Sh::GROUPS * 2 * Sh::BUF * 2, "merge fits");
    float *mo = reinterpret_cast<float *>(&kb[0][0][0]);  // [GROUPS][16 heads][DV]
    float *mml = mo + Sh::GROUPS * 16 * DV;               // [GROUPS][16 heads][2]
    // sink logits of the heads this thread finalises (used when the merge covers the query), loaded
    // together ahead of the exchange
    constexpr int kMit = (16 * DV + Sh::THREADS - 1) / Sh::THREADS;
    float skm[kMit];
#pragma unroll
    for (int it = 0; it < kMit; ++it) {
      const int hh = (tid + it * Sh::THREADS) / DV;
      skm[it] = sink[hh < H ? hh : 0];
    }
    __syncthreads();  // every wave is done reading its chunk buffers
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int cc = 0; cc < CT; ++cc) mo[(grp * 16 + 4 * g + r) * DV + 16 * cc + l16] = oo[cc][r];
    if (g == 0) {
      mml[(grp * 16 + l16) * 2] = item_ok ? mr : -INFINITY;
      mml[(grp * 16 + l16) * 2 + 1] = item_ok ? lr : 0.f;
    }
    __syncthreads();
    const int nsm = NS / Sh::GROUPS;  // merged ranges per query
    const int64_t sitem = wg;         // merged range index: query qm = sitem / nsm
    const int64_t sq = sitem / nsm;
    if (sq >= n_items / NS) return;  // padding workgroup (uniform)
#pragma unroll
    for (int it = 0; it < kMit; ++it) {
      const int e = tid + it * Sh::THREADS;
      if (e >= 16 * DV) break;
      const int h = e / DV, d = e % DV;
      float z = -INFINITY;
#pragma unroll
      for (int gi = 0; gi < Sh::GROUPS; ++gi) z = fmaxf(z, mml[(gi * 16 + h) * 2]);
      float acc = 0.f, lsum = 0.f;
      if (z != -INFINITY) {
#pragma unroll
        for (int gi = 0; gi < Sh::GROUPS; ++gi) {
          const float mg = mml[(gi * 16 + h) * 2];
          const float wgt = mg == -INFINITY ? 0.f : fast_exp2(mg - z);
          lsum += wgt * mml[(gi * 16 + h) * 2 + 1];
          acc += wgt * mo[(gi * 16 + h) * DV + d];
        }
      }
      if (h >= H) continue;
      if (nsm == 1) {
        const float sk = skm[it] * kLog2e;
        const float zz = fmaxf(z, sk);
        float val = 0.f;
        if (zz != -INFINITY) {
          const float ez = z == -INFINITY ? 0.f : exp2f(z - zz);
          const float den = lsum * ez + exp2f(sk - zz);
          val = den > 0.f ? acc * ez / den : 0.f;
        }
        out[(sq * H + h) * DV + d] = f32_to_bf16_rne(val);
      } else {
        part_o[(sitem * H + h) * DV + d] = f32_to_bf16_rne(acc);
        if (d == 0) {
          part_ml[(sitem * H + h) * 2] = z;
          part_ml[(sitem * H + h) * 2 + 1] = lsum;
        }
      }
    }
  };

  // ---- one-wave groups whose workgroup holds consecutive ranges of one query merge in LDS first
  if constexpr (GW == 1 && Sh::GROUPS > 1) {
    if (NS % Sh::GROUPS == 0) {
      merge_groups(o, m_ref, l_run);
      return;
    }
  }
  if (!item_ok) return;
  // ---- finalise: O rows are heads 4g + r; their (max, sum) live in lanes 4g + r
  if (NS == 1) {
    float skv[4];  // sink logits of the lane's output heads, loaded together (one round trip)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hr = gw * 16 + 4 * g + r;
      skv[r] = sink[hr < H ? hr : 0];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hr = gw * 16 + 4 * g + r;
      const float mx = __shfl(m_ref, 4 * g + r, 64);
      const float sm = __shfl(l_run, 4 * g + r, 64);
      if (hr < H) {
        const float sk = skv[r] * kLog2e;
        const float zmax = fmaxf(mx, sk);
        float scale_o = 0.f;
        if (zmax != -INFINITY) {
          const float e = (mx == -INFINITY) ? 0.f : exp2f(mx - zmax);
          const float den = sm * e + exp2f(sk - zmax);
          scale_o = den > 0.f ? e / den : 0.f;
        }
        uint16_t *orow = out + (qm * H + hr) * DV;
#pragma unroll
        for (int cc = 0; cc < CT; ++cc) orow[16 * cc + l16] = f32_to_bf16_rne(o[cc][r] * scale_o);
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hr = gw * 16 + 4 * g + r;
      if (hr < H) {
        uint16_t *po = part_o + (item * H + hr) * DV;
#pragma unroll
        for (int cc = 0; cc < CT; cc += 2) {  // one packed convert per two column tiles
          const uint32_t pk = pack_bf16x2(o[cc][r], o[cc + 1][r]);
          po[16 * cc + l16] = static_cast<uint16_t>(pk & 0xFFFFu);
          po[16 * (cc + 1) + l16] = static_cast<uint16_t>(pk >> 16);
        }
      }
    }
    if (g == 0 && head_ok) {
      float *pml = part_ml + (item * H + head) * 2;
      pml[0] = m_ref;
      pml[1] = l_run;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// MLA-shaped heads (Dqk = 576, Dv = 512, H = 32 NW): one work item per workgroup of NW waves, 32 heads per
// wave (two 16-head tiles), one wave per SIMD.  Each K fragment and each V fragment read from LDS feeds two
// MFMAs (one per head tile), which halves the LDS read traffic per flop of a 16-head wave, and a wave
// alone on its SIMD has 512 registers: the 16 x 512 fp32 O accumulators of both tiles (256) and the q
// B-fragments (144) fit with room left for reading fragments ahead.  The item's row indices are validated
// once into LDS (-1 = invalid), so the only vector-memory operations in the chunk loop are the gathers,
// and an NBUF-deep ring keeps NBUF - 1 chunks in flight with per-wave s_waitcnt vmcnt(n).
template <int NW, int NBUF>
struct MlaShape {
  static constexpr int DQK = 576, DV = 512;
  static constexpr int UPR = DQK / 8;       // 72 16-byte units per row
  static constexpr int UNITS = kKC * UPR;   // 2304 per chunk
  static constexpr int TI = UNITS / 64;     // 36 DMA instructions per chunk
  static constexpr int NJ = TI / NW;        // per wave
  static constexpr int BUF = UNITS * 8;     // bf16 elements per chunk buffer
  static constexpr int QJ = DQK / 32;       // k-steps of the QK MFMA
  static constexpr int CT = DV / 16;        // dv column tiles
  static constexpr int THREADS = 64 * NW;
  static constexpr int KR_MAX = 2048;       // keys per work item (indices staged in LDS)
  // q B-fragments: the first QREG k-steps of both head tiles in VGPRs, the last QL in LDS
  static constexpr int QL = 4;
  static constexpr int QREG = QJ - QL;
  static_assert(TI % NW == 0, "every wave issues the same number of DMA instructions");
  static constexpr int QS = QL > 0 ? NW * QL * 2 * 64 : 1;  // uint4 slots of q in LDS
  static_assert(NBUF * BUF * 2 + KR_MAX * 4 + (QS + NW * 64) * 16 <= 160 * 1024, "LDS budget");
  // same swizzle as SaShape<576, 512, *>: unit u of key k at k*UPR + (u ^ (k & 7)) for the low 3 bits
  __device__ static __forceinline__ int slot(int k, int u_hi, int u_lo) { return k * UPR + u_hi + (u_lo ^ (k & 7)); }
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// O += A B with the accumulator held in AGPRs ("+a"): the compiler would otherwise move the 256 accumulator
// registers between the register files on every iteration.  Inline assembly is invisible to the compiler's
// hazard tracking, so the callers order it with explicit NOPs: VALU writes of A, B or the accumulator
// (P packing, rescaling) are followed by >= 2 wait states before the first such MFMA (mfma_agpr_enter),
// and >= 19 wait states separate the last one from any read of its results (mfma_agpr_leave).
__device__ __forceinline__ void mfma16_agpr(f32x4_t &acc, uint4 a, uint4 b) {
  const u32x4_t va = {a.x, a.y, a.z, a.w}, vb = {b.x, b.y, b.z, b.w};
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(va), "v"(vb));
}

// acc[r] *= s[r] for an accumulator held in AGPRs (AGPRs are not VALU operands): the tuple moves to VGPRs
// and back through the lane's 16-byte LDS slot `slot` (DS writes take AGPR data, ds_read_b128 fills AGPRs),
// so the accumulator is only ever read and defined in the AGPR class; plain copies let the compiler hoist
// the moves of all 256 accumulators out of the rarely taken rescale branch and spill.
__device__ __forceinline__ void scale_agpr(f32x4_t &acc, const float (&s)[4], uint32_t slot) {
  f32x4_t t;
  asm volatile("ds_write_b128 %1, %2\n\ts_waitcnt lgkmcnt(0)\n\tds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
               : "=v"(t)
               : "v"(slot), "a"(acc)
               : "memory");
  t *= f32x4_t{s[0], s[1], s[2], s[3]};
  asm volatile("ds_write_b128 %1, %2\n\ts_waitcnt lgkmcnt(0)\n\tds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
               : "=a"(acc)
               : "v"(slot), "v"(t)
               : "memory");
}

// The same with the accumulator in VGPRs (scores, read by the softmax): fenced by mfma_vgpr_enter/leave.
__device__ __forceinline__ void mfma16_vgpr(f32x4_t &acc, uint4 a, uint4 b) {
  const u32x4_t va = {a.x, a.y, a.z, a.w}, vb = {b.x, b.y, b.z, b.w};
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(va), "v"(vb));
}
__device__ __forceinline__ void mfma_vgpr_enter(f32x4_t (&st)[2][2]) {
  asm volatile("s_nop 2" : "+v"(st[0][0]), "+v"(st[0][1]), "+v"(st[1][0]), "+v"(st[1][1]));
}
__device__ __forceinline__ void mfma_vgpr_leave(f32x4_t (&st)[2][2]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(st[0][0]), "+v"(st[0][1]), "+v"(st[1][0]), "+v"(st[1][1]));
}

// s_waitcnt vmcnt(n) for a run-time n in [0, 2 NJ] (the immediate must be a constant)
template <int N>
__device__ __forceinline__ void wait_vm_le(int n) {
  if constexpr (N > 0) {
    if (n >= N) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N < 63 ? N : 63) : "memory");
      return;
    }
    wait_vm_le<N - 1>(n);
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// Hazard fences for mfma16_agpr over the O accumulators o[2][CT] (tied, so nothing that writes or reads
// them moves across): 2 wait states after the VALU writes of P / O, 24 before reading the results.
template <int CT>
__device__ __forceinline__ void mfma_agpr_enter(f32x4_t (&o)[2][CT], uint4 (&pa)[2]) {
  asm volatile("s_nop 2" : "+v"(pa[0].x), "+v"(pa[0].y), "+v"(pa[0].z), "+v"(pa[0].w), "+v"(pa[1].x),
               "+v"(pa[1].y), "+v"(pa[1].z), "+v"(pa[1].w));
#pragma unroll
  for (int c = 0; c < CT; c += 4)
    asm volatile("" : "+a"(o[0][c]), "+a"(o[0][c + 1]), "+a"(o[0][c + 2]), "+a"(o[0][c + 3]), "+a"(o[1][c]),
                 "+a"(o[1][c + 1]), "+a"(o[1][c + 2]), "+a"(o[1][c + 3]));
}
// The MFMAs that wrote O have finished 24 wait states after this: every one of them is issued before it
// (the empty statements take all of O as inputs and are ordered with the NOPs), and nothing is tied, so
// no register copy of O is needed to set it up.  At the end of each chunk this keeps register copies that
// the compiler places at the loop exit or back edge behind the NOPs.
template <int CT>
__device__ __forceinline__ void mfma_agpr_settle(const f32x4_t (&o)[2][CT]) {
#pragma unroll
  for (int c = 0; c < CT; c += 4)
    asm volatile("" ::"a"(o[0][c]), "a"(o[0][c + 1]), "a"(o[0][c + 2]), "a"(o[0][c + 3]), "a"(o[1][c]),
                 "a"(o[1][c + 1]), "a"(o[1][c + 2]), "a"(o[1][c + 3]));
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}
template <int CT>
__device__ __forceinline__ void mfma_agpr_leave(f32x4_t (&o)[2][CT]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int c = 0; c < CT; c += 4)
    asm volatile("" : "+a"(o[0][c]), "+a"(o[0][c + 1]), "+a"(o[0][c + 2]), "+a"(o[0][c + 3]), "+a"(o[1][c]),
                 "+a"(o[1][c + 1]), "+a"(o[1][c + 2]), "+a"(o[1][c + 3]));
}

// Partial ranges of the MLA kernel in its own register layout ("fragment layout"): range `item`, wave w, head tile
// ht, pair of column tiles cp = cc / 2, lane l = l16 + 16 g holds the 16-byte unit
//   bf16 of O[head 32 w + 16 ht + 4 g + r][column 16 cc + l16] for (cc, r) = (2 cp, 0..3), (2 cp + 1, 0..3),
// units ordered [item][w][ht][cp][lane] (the same bytes as row-major partials: H = 32 NW heads x 512 columns).
__host__ __device__ inline int64_t mla_frag_offset(int64_t item, int NW, int w, int ht, int cp, int lane) {
  return (((item * NW + w) * 2 + ht) * 16 + cp) * 64 + lane;
}

template <int NW, int NBUF>
__global__ __launch_bounds__(64 * NW, 1) void sparse_attn_mla_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ kv, const float *__restrict__ sink,
    const int32_t *__restrict__ idx, uint16_t *__restrict__ out, uint16_t *__restrict__ part_o,
    float *__restrict__ part_ml, int64_t M, int H, int64_t N, int64_t K, int NS, int KR, float scale_log2) {
  using Sh = MlaShape<NW, NBUF>;
  constexpr int QJ = Sh::QJ, QREG = Sh::QREG, QL = Sh::QL, CT = Sh::CT, UPR = Sh::UPR, NJ = Sh::NJ;
  __shared__ __attribute__((aligned(16))) uint16_t kb[NBUF][Sh::BUF];
  __shared__ __attribute__((aligned(16))) uint4 qs[Sh::QS];  // [wave][k-step - QREG][head tile][lane]
  __shared__ __attribute__((aligned(16))) uint4 rsc[NW][64];  // rescale bounce slots
  __shared__ int32_t sidx[Sh::KR_MAX];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  // one item per workgroup (grid = items); the ranges of one query share an XCD (block id mod 8)
  const int64_t nblk = gridDim.x;
  const int64_t item = (nblk % 8 == 0) ? (blockIdx.x % 8) * (nblk / 8) + blockIdx.x / 8 : blockIdx.x;
  const int64_t qm = item / NS;
  const int split = static_cast<int>(item % NS);
  const int64_t b = qm / M;
  const int k_begin = split * KR;
  const int k_end = k_begin + KR < K ? k_begin + KR : static_cast<int>(K);
  const int nch = (k_end - k_begin + kKC - 1) / kKC;  // >= 1: every range of the plan is non-empty
  const global_ptr<const uint16_t> kvb = uniform_ptr(kv + b * N * Sh::DQK);

  // ---- the item's row indices and the q B-fragments are loaded together (one round trip): the indices
  // first, unrolled (wave-uniform guards, positions clamped into the range), so that staging them waits for
  // them alone; q: Q[head][32j + 8g .. +7] with head = 32 wave + 16 ht + l16 for both head tiles, all in VGPRs
  // (the k-steps past QREG, if any, in LDS)
  constexpr int kIPT = (Sh::KR_MAX + Sh::THREADS - 1) / Sh::THREADS;
  const int ntot = nch * kKC;  // <= KR_MAX (host-checked range length, rounded up to whole chunks)
  int32_t iraw[kIPT];
  {
    const int32_t *irow = idx + qm * K;
#pragma unroll
    for (int i = 0; i < kIPT; ++i) {
      const int pos = k_begin + tid + i * Sh::THREADS;
      iraw[i] = -1;
      if (i * Sh::THREADS < ntot) iraw[i] = irow[pos < k_end ? pos : k_end - 1];
    }
  }
  uint4 qf[2][QREG];
#pragma unroll
  for (int ht = 0; ht < 2; ++ht) {
    const uint16_t *qrow = q + (qm * H + 32 * wave + 16 * ht + l16) * Sh::DQK + 8 * g;
#pragma unroll
    for (int j = 0; j < QJ; ++j) {
      const uint4 v = *reinterpret_cast<const uint4 *>(qrow + 32 * j);
      if (j < QREG) qf[ht][j < QREG ? j : 0] = v;
      else qs[((wave * QL + (j < QREG ? 0 : j - QREG)) * 2 + ht) * 64 + lane] = v;
    }
  }
  // staged validated (-1 = outside the range or not in [0, N))
#pragma unroll
  for (int i = 0; i < kIPT; ++i) {
    const int t = tid + i * Sh::THREADS;
    if (t < ntot) sidx[t] = (k_begin + t < k_end && iraw[i] >= 0 && iraw[i] < N) ? iraw[i] : -1;
  }
  // the q loads complete here, not at their first use inside the loop (where the wait would also drain
  // the gathers in flight on every iteration)
#pragma unroll
  for (int ht = 0; ht < 2; ++ht)
#pragma unroll
    for (int j = 0; j < QREG; ++j)
      asm volatile("" : "+v"(qf[ht][j].x), "+v"(qf[ht][j].y), "+v"(qf[ht][j].z), "+v"(qf[ht][j].w));
  __syncthreads();  // indices (and q's LDS part) staged

  // DMA slot 64 (wave + NW i) + lane of a chunk holds unit (slot % 72) ^ (key & 7) of key slot / 72
  const uint32_t kb_lds = __builtin_amdgcn_readfirstlane(lds_addr(&kb[0][0]));
  auto issue = [&](int c) {
    const int buf = c % NBUF;
    // one-wave workgroups (36 gathers) redo the slot arithmetic per chunk (opaque lane): kept live across
    // the loop, their per-gather offsets would take 72 registers
    int ln = lane;
    if constexpr (NW == 1) asm volatile("" : "+v"(ln));
    // index reads in batches of a divisor of NJ (36, 18, 12, 9): one LDS latency per batch
    constexpr int BATCH = NJ <= 12 ? NJ : 9;
    static_assert(NJ % BATCH == 0, "every batch lies inside the wave's NJ gathers");
#pragma unroll
    for (int i0 = 0; i0 < NJ; i0 += BATCH) {
      int32_t r[BATCH];
#pragma unroll
      for (int i = 0; i < BATCH; ++i) r[i] = sidx[c * kKC + (64 * (wave + NW * (i0 + i)) + ln) / UPR];
#pragma unroll
      for (int i = 0; i < BATCH; ++i) {
        const int jj = wave + NW * (i0 + i);
        const int sl = 64 * jj + ln;
        const int key = sl / UPR;
        const uint32_t voff =
            static_cast<uint32_t>(r[i] < 0 ? 0 : r[i]) * (Sh::DQK * 2) + ((sl % UPR) ^ (key & 7)) * 16;
        dma16((const void *)kvb, voff, kb_lds + (buf * Sh::BUF + 64 * jj * 8) * 2);
      }
    }
  };
  const int npre = nch < NBUF - 1 ? nch : NBUF - 1;
  for (int c = 0; c < npre; ++c) issue(c);

  // per-lane LDS element offsets (see SaShape): QK key 16t + l16, unit 4j + g (two low-unit patterns);
  // PV transpose reads keys 4g + (l16 >> 2) (+16), unit 2cc + ((l16 & 3) >> 1) (four patterns)
  int qk_off[2][2], pv_off[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int p = 0; p < 2; ++p) qk_off[t][p] = Sh::slot(16 * t + l16, 0, 4 * p + g) * 8;
    const int kv_key = 4 * g + (l16 >> 2) + 16 * t;
#pragma unroll
    for (int p = 0; p < 4; ++p) pv_off[t][p] = Sh::slot(kv_key, 0, 2 * p + ((l16 & 3) >> 1)) * 8 + 4 * (l16 & 1);
  }

  float m_ref[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};  // per head (lane l16), replicated over g
  f32x4_t o[2][CT];
#pragma unroll
  for (int ht = 0; ht < 2; ++ht)
#pragma unroll
    for (int c = 0; c < CT; ++c) o[ht][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int c = 0; c < nch; ++c) {
    // this wave's part of chunk c has landed once at most (chunks issued after it) x NJ gathers remain
    const int later = (nch - 1 - c) < (NBUF - 2) ? (nch - 1 - c) : (NBUF - 2);
    wait_vm_le<(NBUF - 2) * NJ>(later * NJ);
    __syncthreads();  // everyone's part of chunk c (and of q in LDS) is in place; chunk c - 1's buffer is free
    if (c + NBUF - 1 < nch) issue(c + NBUF - 1);
    const uint32_t vm = static_cast<uint32_t>(__builtin_amdgcn_ballot_w64(sidx[c * kKC + (lane & 31)] >= 0));
    const uint16_t *kbp = kb[c % NBUF];

    // ---- S^T = K Q^T: key tiles t, head tiles ht; each K fragment feeds both head tiles
    f32x4_t st[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int ht = 0; ht < 2; ++ht) st[t][ht] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    mfma_vgpr_enter(st);
#pragma unroll
    for (int j = 0; j < QJ; ++j) {
      const int jl = j < QREG ? 0 : j - QREG;
      const uint4 b0 = j < QREG ? qf[0][j < QREG ? j : 0] : qs[((wave * QL + jl) * 2 + 0) * 64 + lane];
      const uint4 b1 = j < QREG ? qf[1][j < QREG ? j : 0] : qs[((wave * QL + jl) * 2 + 1) * 64 + lane];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint4 a = *reinterpret_cast<const uint4 *>(kbp + qk_off[t][j & 1] + ((4 * j) & ~7) * 8);
        mfma16_vgpr(st[t][0], a, b0);
        mfma16_vgpr(st[t][1], a, b1);
      }
    }
    mfma_vgpr_leave(st);
    // ---- online softmax per head tile (lane: head l16, keys 16t + 4g + r)
    const uint32_t vbits = vm >> (4 * g);
    float cmax[2];
#pragma unroll
    for (int ht = 0; ht < 2; ++ht) {
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if ((vbits >> (16 * t + r)) & 1u) mx = fmaxf(mx, st[t][ht][r] * scale_log2);
      cmax[ht] = rows_max(mx);
    }
    const bool need0 = cmax[0] > m_ref[0] + kRescaleTau, need1 = cmax[1] > m_ref[1] + kRescaleTau;
    if (__builtin_amdgcn_ballot_w64(need0 || need1) != 0ull) {
#pragma unroll
      for (int ht = 0; ht < 2; ++ht) {
        const bool need = ht == 0 ? need0 : need1;
        // O is still zero for heads without a finite reference yet (the first valid chunk), so the
        // accumulators are rescaled only when some head moves a finite reference
        const bool move = need && m_ref[ht] != -INFINITY;
        const float m_new = need ? cmax[ht] : m_ref[ht];
        const float alpha = need ? (m_ref[ht] == -INFINITY ? 0.f : fast_exp2(m_ref[ht] - m_new)) : 1.f;
        l_run[ht] *= alpha;
        m_ref[ht] = m_new;
        if (__builtin_amdgcn_ballot_w64(move) != 0ull) {
          float ar[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * g + r, 64);
          const uint32_t slot = lds_addr(&rsc[wave][lane]);
#pragma unroll
          for (int cc = 0; cc < CT; ++cc) scale_agpr(o[ht][cc], ar, slot);
        }
      }
    }
    uint4 pa[2];
#pragma unroll
    for (int ht = 0; ht < 2; ++ht) {
      float p[8], csum = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool ok = (vbits >> (16 * (i >> 2) + (i & 3))) & 1u;
        p[i] = ok ? fast_exp2(st[i >> 2][ht][i & 3] * scale_log2 - m_ref[ht]) : 0.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) csum += p[i];
      l_run[ht] += rows_sum(csum);
      pa[ht] = make_uint4(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                          pack_bf16x2(p[6], p[7]));
    }
    // ---- O += P V; each V fragment feeds both head tiles
    mfma_agpr_enter(o, pa);
#pragma unroll
    for (int cc = 0; cc < CT; ++cc) {
      const int hi = ((2 * cc) & ~7) * 8;
      const uint2 b0 = lds_read_tr16(kbp + pv_off[0][cc & 3] + hi);
      const uint2 b1 = lds_read_tr16(kbp + pv_off[1][cc & 3] + hi);
      const uint4 vb = make_uint4(b0.x, b0.y, b1.x, b1.y);
      mfma16_agpr(o[0][cc], pa[0], vb);
      mfma16_agpr(o[1][cc], pa[1], vb);
    }
    mfma_agpr_settle(o);
  }
  mfma_agpr_leave(o);

  // ---- finalise (one range per query: sink added, bf16 output) or write the partial range
  const int64_t obase = NS == 1 ? qm : item;
  float skv[2][4];  // sink logits of the lane's output heads, loaded together (one round trip)
#pragma unroll
  for (int ht = 0; ht < 2; ++ht)
#pragma unroll
    for (int r = 0; r < 4; ++r) skv[ht][r] = NS == 1 ? sink[32 * wave + 16 * ht + 4 * g + r] : 0.f;
#pragma unroll
  for (int ht = 0; ht < 2; ++ht) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hr = 32 * wave + 16 * ht + 4 * g + r;
      const float mx = __shfl(m_ref[ht], 4 * g + r, 64);
      const float sm = __shfl(l_run[ht], 4 * g + r, 64);
      float scale_o = 1.f;
      if (NS == 1) {
        const float sk = skv[ht][r] * kLog2e;
        const float zmax = fmaxf(mx, sk);
        scale_o = 0.f;
        if (zmax != -INFINITY) {
          const float e = (mx == -INFINITY) ? 0.f : exp2f(mx - zmax);
          const float den = sm * e + exp2f(sk - zmax);
          scale_o = den > 0.f ? e / den : 0.f;
        }
      }
      if (NS == 1) {
        uint16_t *orow = out + (obase * H + hr) * Sh::DV;
#pragma unroll
        for (int cc = 0; cc < CT; cc += 2) {  // one packed convert per two column tiles
          const uint32_t pk = pack_bf16x2(o[ht][cc][r] * scale_o, o[ht][cc + 1][r] * scale_o);
          orow[16 * cc + l16] = static_cast<uint16_t>(pk & 0xFFFFu);
          orow[16 * (cc + 1) + l16] = static_cast<uint16_t>(pk >> 16);
        }
      }
    }
    if (NS > 1) {
      // the partial range in the fragment layout (mla_frag_offset): one 16-byte store per lane and pair of column
      // tiles, the wave's 64 lanes writing 1 KiB contiguously (row-major rows would take 2-byte stores)
      uint4 *pf = reinterpret_cast<uint4 *>(part_o) + mla_frag_offset(item, NW, wave, ht, 0, lane);
#pragma unroll
      for (int cc = 0; cc < CT; cc += 2)
        pf[(cc / 2) * 64] = make_uint4(pack_bf16x2(o[ht][cc][0], o[ht][cc][1]), pack_bf16x2(o[ht][cc][2], o[ht][cc][3]),
                                       pack_bf16x2(o[ht][cc + 1][0], o[ht][cc + 1][1]),
                                       pack_bf16x2(o[ht][cc + 1][2], o[ht][cc + 1][3]));
    }
    if (NS > 1 && g == 0) {
      float *pml = part_ml + (item * H + 32 * wave + 16 * ht + l16) * 2;
      pml[0] = m_ref[ht];
      pml[1] = l_run[ht];
    }
  }
}


// 16-byte units (two column tiles each) per lane and range: one unit per lane gives 4096 waves at config 5 (two
// units: 2048 waves, 0.3 us slower, within the noise)
constexpr int kMlaCombineUnits = 1;

// One DPP lane movement within each 16-lane row: CTRL = 0x150 + n broadcasts lane n of the row (row_newbcast),
// 0x120 + n rotates the row by n lanes (row_ror).
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// row_newbcast of lane n, for an n that is a constant once the caller's loop is unrolled
__device__ __forceinline__ float row_bcast(float v, int n) {
  switch (n) {
    case 0: return dpp_row<0x150>(v);
    case 1: return dpp_row<0x151>(v);
    case 2: return dpp_row<0x152>(v);
    case 3: return dpp_row<0x153>(v);
    case 4: return dpp_row<0x154>(v);
    case 5: return dpp_row<0x155>(v);
    case 6: return dpp_row<0x156>(v);
    case 7: return dpp_row<0x157>(v);
    case 8: return dpp_row<0x158>(v);
    case 9: return dpp_row<0x159>(v);
    case 10: return dpp_row<0x15A>(v);
    case 11: return dpp_row<0x15B>(v);
    case 12: return dpp_row<0x15C>(v);
    case 13: return dpp_row<0x15D>(v);
    case 14: return dpp_row<0x15E>(v);
    case 15: return dpp_row<0x15F>(v);
    default: return v;
  }
}

// Merge of the MLA kernel's NS partial ranges (fragment layout) with the sink.  A wave owns (query, w, ht, a slice e
// of UPW units): lane (l16, g) accumulates heads hb + 4 g + r (hb = 32 w + 16 ht, r = 0..3) over the column tiles
// 2 UPW e .. 2 UPW e + 2 UPW - 1, so every partial read is a 1 KiB contiguous wave access.  The (max, sum) pairs of
// a group of 8 ranges x the wave's 16 heads are one float4 per lane, laid out so that each 16-lane row holds its own
// heads: lane (l16, g) loads range l16 / 2, heads hb + 4 g + 2 (l16 & 1) + {0, 1}.  The weights are formed there, the
// maxima and denominators are reduced over the row's ranges by row rotations, and each weight reaches the
// accumulating lanes by one row broadcast (DPP: no LDS traffic, no address arithmetic).  Output: lane pairs
// (l16, l16 ^ 1) swap two of their four heads, so each lane writes two adjacent columns of two heads as 4-byte stores.
__global__ __launch_bounds__(256) void sparse_attn_mla_combine_kernel(const uint4 *__restrict__ part_f,
                                                                     const float *__restrict__ part_ml,
                                                                     const float *__restrict__ sink,
                                                                     uint16_t *__restrict__ out, int64_t n_q, int NW,
                                                                     int NS) {
  constexpr int DV = 512, UPW = kMlaCombineUnits, EPW = 16 / UPW, kGroup = 8;
  const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
  // XCD placement of the attention kernel: a query's ranges were written on one XCD (block id mod 8)
  const int64_t nblk = gridDim.x;
  const int64_t lb = (nblk % 8 == 0) ? (blockIdx.x % 8) * (nblk / 8) + blockIdx.x / 8 : blockIdx.x;
  const int64_t wv = lb * 4 + (threadIdx.x >> 6);  // (query, w, ht, e)
  const int64_t per_q = static_cast<int64_t>(NW) * 2 * EPW;
  if (wv >= n_q * per_q) return;  // uniform per wave
  const int64_t qm = wv / per_q;
  const int rem = static_cast<int>(wv % per_q);
  const int w = rem / (2 * EPW), ht = (rem / EPW) % 2, e = rem % EPW;
  const int H = 32 * NW;
  const int hb = 32 * w + 16 * ht;
  const int ls = l16 >> 1, hp = hb + 4 * g + 2 * (l16 & 1);  // loader: range ls of a group, heads hp, hp + 1
  const float *mlq = part_ml + (qm * NS * H + hp) * 2;
  auto load_ml = [&](int s0) {
    const int sr = s0 + ls;
    const float4 v = *reinterpret_cast<const float4 *>(mlq + static_cast<int64_t>(sr < NS ? sr : NS - 1) * H * 2);
    return sr < NS ? v : make_float4(-INFINITY, 0.f, -INFINITY, 0.f);
  };
  const uint4 *pfq = part_f + mla_frag_offset(qm * NS, NW, w, ht, UPW * e, lane);
  const int64_t range_units = static_cast<int64_t>(NW) * 2 * 16 * 64;  // 16-byte units of one range
  auto load_units = [&](int s0, uint4 (&fv)[kGroup][UPW]) {
#pragma unroll
    for (int s = 0; s < kGroup; ++s) {
      const uint4 *pf = pfq + (s0 + s < NS ? s0 + s : NS - 1) * range_units;
#pragma unroll
      for (int u = 0; u < UPW; ++u) fv[s][u] = pf[64 * u];
    }
  };
  // every load of the first group goes out before the first wait
  const float4 ml0 = load_ml(0);
  uint4 f0[kGroup][UPW];
  load_units(0, f0);
  const float sk0 = sink[hp] * kLog2e, sk1 = sink[hp + 1] * kLog2e;
  __builtin_amdgcn_sched_barrier(0);  // keep the loads above the reduction
  // the largest logit of the loader's two heads: the ranges' maxima (rotations over the row's 8 ranges) and the sink
  float z0 = ml0.x, z1 = ml0.z;
  for (int s0 = kGroup; s0 < NS; s0 += kGroup) {
    const float4 v = load_ml(s0);
    z0 = fmaxf(z0, v.x);
    z1 = fmaxf(z1, v.z);
  }
  z0 = fmaxf(z0, dpp_row<0x122>(z0));
  z1 = fmaxf(z1, dpp_row<0x122>(z1));
  z0 = fmaxf(z0, dpp_row<0x124>(z0));
  z1 = fmaxf(z1, dpp_row<0x124>(z1));
  z0 = fmaxf(fmaxf(z0, dpp_row<0x128>(z0)), sk0);
  z1 = fmaxf(fmaxf(z1, dpp_row<0x128>(z1)), sk1);
  float acc[4][2 * UPW];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int i = 0; i < 2 * UPW; ++i) acc[r][i] = 0.f;
  float dp0 = 0.f, dp1 = 0.f;  // the loader's share of the denominators
  // one group: weights on the loaders, then each range's units weighted per head (head hb + 4 g + r: lane
  // 2 s + (r >> 1) of the row, its weight of head r & 1)
  auto group = [&](int s0, const float4 &v, const uint4 (&fv)[kGroup][UPW]) {
    const float w0 = (v.x == -INFINITY || z0 == -INFINITY) ? 0.f : exp2f(v.x - z0);
    const float w1 = (v.z == -INFINITY || z1 == -INFINITY) ? 0.f : exp2f(v.z - z1);
    dp0 += w0 * v.y;
    dp1 += w1 * v.w;
#pragma unroll
    for (int s = 0; s < kGroup; ++s) {
      if (s0 + s >= NS) break;  // uniform
      const float ws[4] = {row_bcast(w0, 2 * s), row_bcast(w1, 2 * s), row_bcast(w0, 2 * s + 1),
                           row_bcast(w1, 2 * s + 1)};
#pragma unroll
      for (int u = 0; u < UPW; ++u) {
        const uint32_t x[4] = {fv[s][u].x, fv[s][u].y, fv[s][u].z, fv[s][u].w};  // (tile 2u: r 0 1, r 2 3), ...
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          acc[0][2 * u + t] += ws[0] * __builtin_bit_cast(float, x[2 * t] << 16);
          acc[1][2 * u + t] += ws[1] * __builtin_bit_cast(float, x[2 * t] & 0xFFFF0000u);
          acc[2][2 * u + t] += ws[2] * __builtin_bit_cast(float, x[2 * t + 1] << 16);
          acc[3][2 * u + t] += ws[3] * __builtin_bit_cast(float, x[2 * t + 1] & 0xFFFF0000u);
        }
      }
    }
  };
  group(0, ml0, f0);
  for (int s0 = kGroup; s0 < NS; s0 += kGroup) {
    const float4 v = load_ml(s0);
    uint4 fv[kGroup][UPW];
    load_units(s0, fv);
    group(s0, v, fv);
  }
  dp0 += dpp_row<0x122>(dp0);
  dp1 += dpp_row<0x122>(dp1);
  dp0 += dpp_row<0x124>(dp0);
  dp1 += dpp_row<0x124>(dp1);
  dp0 += dpp_row<0x128>(dp0);
  dp1 += dpp_row<0x128>(dp1);
  const float den0 = dp0 + (z0 == -INFINITY ? 0.f : exp2f(sk0 - z0));
  const float den1 = dp1 + (z1 == -INFINITY ? 0.f : exp2f(sk1 - z1));
  const float iv0 = den0 > 0.f ? 1.f / den0 : 0.f, iv1 = den1 > 0.f ? 1.f / den1 : 0.f;
  const float inv[4] = {dpp_row<0x150>(iv0), dpp_row<0x150>(iv1), dpp_row<0x151>(iv0), dpp_row<0x151>(iv1)};
  // even l16 keeps heads r = 0, 2 and receives its odd neighbour's; odd l16 keeps r = 1, 3
  const bool odd = (l16 & 1) != 0;
  uint16_t *obase = out + (qm * H + hb + 4 * g) * DV + 16 * (2 * UPW * e) + (l16 & ~1);
#pragma unroll
  for (int i = 0; i < 2 * UPW; ++i) {
    const float v0 = acc[0][i] * inv[0], v1 = acc[1][i] * inv[1], v2 = acc[2][i] * inv[2], v3 = acc[3][i] * inv[3];
    const float y0 = dpp_row<0xB1>(odd ? v0 : v1);  // quad_perm [1,0,3,2]: the lane's neighbour l16 ^ 1
    const float y1 = dpp_row<0xB1>(odd ? v2 : v3);
    const int ra = odd ? 1 : 0;  // rows ra and ra + 2
    const uint32_t wa = odd ? pack_bf16x2(y0, v1) : pack_bf16x2(v0, y0);
    const uint32_t wb = odd ? pack_bf16x2(y1, v3) : pack_bf16x2(v2, y1);
    *reinterpret_cast<uint32_t *>(obase + ra * DV + 16 * i) = wa;
    *reinterpret_cast<uint32_t *>(obase + (ra + 2) * DV + 16 * i) = wb;
  }
}

// Merge the NS partial ranges of one (query, head) row with the sink: one wave per row, lane s reads
// range s's (max, sum); every lane then accumulates DV/64 columns over the ranges.  The first PRE ranges'
// columns are loaded ahead of the reduction (PRE >= NS where NS <= 8, so no load is spent on a clamped range).
template <int DV, int PRE>
__global__ __launch_bounds__(256) void sparse_attn_combine_kernel(const uint16_t *__restrict__ part_o,
                                                                 const float *__restrict__ part_ml,
                                                                 const float *__restrict__ sink,
                                                                 uint16_t *__restrict__ out, int64_t rows, int H,
                                                                 int NS) {
  constexpr int CPL = DV / 64;  // columns per lane
  const int lane = threadIdx.x & 63;
  // the same XCD placement as the attention kernels (workgroup i on XCD i mod 8, consecutive logical
  // blocks on one XCD): a query's rows are merged on the XCD whose L2 received its partial ranges
  const int64_t nblk = gridDim.x;
  const int64_t lb = (nblk % 8 == 0) ? (blockIdx.x % 8) * (nblk / 8) + blockIdx.x / 8 : blockIdx.x;
  const int64_t row = lb * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // uniform per wave
  const int64_t qm = row / H;
  const int h = static_cast<int>(row % H);
  // every load of the first kPre ranges goes out before the first wait: the sink, the ranges' (max, sum)
  // (lane s: range min(s, NS - 1), masked below) and their O columns, which do not depend on them
  constexpr int kPre = PRE;
  const float sk_raw = sink[h];
  const float *ml = part_ml + ((qm * NS + (lane < NS ? lane : NS - 1)) * H + h) * 2;
  const float m_raw = ml[0], l_raw = ml[1];
  const uint16_t *po = part_o + (qm * NS * H + h) * DV + lane * CPL;
  uint32_t pre[kPre][CPL / 2];
#pragma unroll
  for (int s = 0; s < kPre; ++s) {
    const uint32_t *src = reinterpret_cast<const uint32_t *>(po + static_cast<int64_t>(s < NS ? s : NS - 1) * H * DV);
#pragma unroll
    for (int i = 0; i < CPL; i += 2) pre[s][i / 2] = src[i / 2];
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the loads above: the scheduler would sink them below the reduction
  const float sk = sk_raw * kLog2e;
  const float m = lane < NS ? m_raw : -INFINITY, l = lane < NS ? l_raw : 0.f;
  float z = m;
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) z = fmaxf(z, __shfl_xor(z, d, 64));
  z = fmaxf(z, sk);
  const float w = (m == -INFINITY || z == -INFINITY) ? 0.f : exp2f(m - z);
  float den = w * l;
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) den += __shfl_xor(den, d, 64);
  if (z != -INFINITY) den += exp2f(sk - z);
  float acc[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) acc[i] = 0.f;
  // empty ranges have w = 0 and O = 0, so every range is accumulated without a branch (ranges past NS in
  // the preloaded block get weight 0)
#pragma unroll
  for (int s = 0; s < kPre; ++s) {
    const float ws = s < NS ? __shfl(w, s, 64) : 0.f;
#pragma unroll
    for (int i = 0; i < CPL; i += 2) {
      const uint32_t v = pre[s][i / 2];
      acc[i] += ws * __builtin_bit_cast(float, v << 16);
      acc[i + 1] += ws * __builtin_bit_cast(float, v & 0xFFFF0000u);
    }
  }
#pragma unroll 8
  for (int s = kPre; s < NS; ++s) {
    const float ws = __shfl(w, s, 64);
    const uint32_t *src = reinterpret_cast<const uint32_t *>(po + static_cast<int64_t>(s) * H * DV);
#pragma unroll
    for (int i = 0; i < CPL; i += 2) {
      const uint32_t v = src[i / 2];
      acc[i] += ws * __builtin_bit_cast(float, v << 16);
      acc[i + 1] += ws * __builtin_bit_cast(float, v & 0xFFFF0000u);
    }
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  uint16_t *orow = out + row * DV + lane * CPL;
#pragma unroll
  for (int i = 0; i < CPL; i += 2)
    *reinterpret_cast<uint32_t *>(orow + i) = pack_bf16x2(acc[i] * inv, acc[i + 1] * inv);
}

template <int DV>
int launch_combine(const uint16_t *part_o, const float *part_ml, const float *sink, uint16_t *out, int64_t rows, int H,
                   int NS, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ceil_div(rows, 4))), block(256);
  if (NS <= 2)
    hipLaunchKernelGGL((sparse_attn_combine_kernel<DV, 2>), grid, block, 0, stream, part_o, part_ml, sink, out, rows, H, NS);
  else if (NS <= 4)
    hipLaunchKernelGGL((sparse_attn_combine_kernel<DV, 4>), grid, block, 0, stream, part_o, part_ml, sink, out, rows, H, NS);
  else
    hipLaunchKernelGGL((sparse_attn_combine_kernel<DV, 8>), grid, block, 0, stream, part_o, part_ml, sink, out, rows, H, NS);
  KS_CHECK_LAUNCH("sparse_attn_combine_kernel");
  return KS_OK;
}

template <int DQK, int DV, int GW>
int launch_sa_gw(const uint16_t *q, const uint16_t *kv, const float *sink, const int32_t *idx, uint16_t *out,
                 int64_t B, int64_t M, int64_t H, int64_t N, int64_t K, float scale, void *ws, hipStream_t stream) {
  using Sh = SaShape<DQK, DV, GW>;
  const SaSplit sp = split_plan(B, M, H, K);
  const int64_t n_items = B * M * sp.ns;
  // split partials: (max, sum) pairs in fp32, then the unnormalised O rows in bf16 (16-byte aligned: H is a
  // multiple of 16)
  uint16_t *part_o = nullptr;
  float *part_ml = nullptr;
  if (sp.ns > 1) {
    part_ml = static_cast<float *>(ws);
    part_o = reinterpret_cast<uint16_t *>(part_ml + n_items * H * 2);
  }
  const int64_t blocks = ceil_div(n_items, Sh::GROUPS);
  hipLaunchKernelGGL((sparse_attn_kernel<DQK, DV, GW>), dim3(static_cast<unsigned>(blocks)), dim3(Sh::THREADS), 0,
                     stream, q, kv, sink, idx, out, part_o, part_ml, n_items, M, static_cast<int>(H), N, K, sp.ns,
                     sp.kr, scale * kLog2e);
  KS_CHECK_LAUNCH("sparse_attn_kernel");
  // one-wave groups merge the ranges of a workgroup in LDS when a workgroup holds whole ranges of a query
  const bool merged = GW == 1 && Sh::GROUPS > 1 && sp.ns % Sh::GROUPS == 0;
  const int ns_left = merged ? sp.ns / Sh::GROUPS : sp.ns;
  if (ns_left > 1) return launch_combine<DV>(part_o, part_ml, sink, out, B * M * H, static_cast<int>(H), ns_left, stream);
  return KS_OK;
}

// MLA kernel: H = 32 NW heads (NW <= 4), every range at most MlaShape::KR_MAX keys, ~one item per CU
constexpr int kMlaTargetItems = 256;
constexpr int kMlaBuffers = 3;
inline bool use_mla(int64_t Dqk, int64_t Dv, int64_t H, int64_t K) {
  return Dqk == 576 && Dv == 512 && H % 32 == 0 && H <= 128 && K <= 64 * 2048;
}
inline SaSplit mla_plan(int64_t B, int64_t M, int64_t K) {
  const int64_t chunks = (K + kKC - 1) / kKC;
  const int64_t bm = B * M > 0 ? B * M : 1;
  int64_t ns = (kMlaTargetItems + bm - 1) / bm;
  const int64_t cap = chunks / kMinChunks > 1 ? chunks / kMinChunks : 1;
  if (ns > cap) ns = cap;
  if (ns > 64) ns = 64;
  const int64_t ns_min = (K + 2047) / 2048;  // ranges of at most 2048 keys (staged indices)
  if (ns < ns_min) ns = ns_min;
  if (ns < 1) ns = 1;
  const int64_t kr = ((chunks + ns - 1) / ns) * kKC;
  return SaSplit{static_cast<int>((K + kr - 1) / kr), static_cast<int>(kr)};
}

template <int NW>
int launch_mla_nw(const uint16_t *q, const uint16_t *kv, const float *sink, const int32_t *idx, uint16_t *out,
                  int64_t B, int64_t M, int64_t H, int64_t N, int64_t K, float scale, void *ws, hipStream_t stream) {
  using Sh = MlaShape<NW, kMlaBuffers>;
  const SaSplit sp = mla_plan(B, M, K);
  const int64_t n_items = B * M * sp.ns;
  uint16_t *part_o = nullptr;
  float *part_ml = nullptr;
  if (sp.ns > 1) {
    part_ml = static_cast<float *>(ws);
    part_o = reinterpret_cast<uint16_t *>(part_ml + n_items * H * 2);
  }
  hipLaunchKernelGGL((sparse_attn_mla_kernel<NW, kMlaBuffers>), dim3(static_cast<unsigned>(n_items)),
                     dim3(Sh::THREADS), 0, stream, q, kv, sink, idx, out, part_o, part_ml, M, static_cast<int>(H), N,
                     K, sp.ns, sp.kr, scale * kLog2e);
  KS_CHECK_LAUNCH("sparse_attn_mla_kernel");
  if (sp.ns > 1) {
    // waves of (query, wave of the attention kernel, head tile, column tiles of kMlaCombineUnits units)
    const int64_t waves = B * M * NW * 2 * (16 / kMlaCombineUnits);
    hipLaunchKernelGGL(sparse_attn_mla_combine_kernel, dim3(static_cast<unsigned>(ceil_div(waves, 4))), dim3(256), 0,
                       stream, reinterpret_cast<const uint4 *>(part_o), part_ml, sink, out, B * M, NW, sp.ns);
    KS_CHECK_LAUNCH("sparse_attn_mla_combine_kernel");
  }
  return KS_OK;
}

int launch_mla(const uint16_t *q, const uint16_t *kv, const float *sink, const int32_t *idx, uint16_t *out, int64_t B,
               int64_t M, int64_t H, int64_t N, int64_t K, float scale, void *ws, hipStream_t stream) {
  switch (H / 32) {
    case 1: return launch_mla_nw<1>(q, kv, sink, idx, out, B, M, H, N, K, scale, ws, stream);
    case 2: return launch_mla_nw<2>(q, kv, sink, idx, out, B, M, H, N, K, scale, ws, stream);
    case 3: return launch_mla_nw<3>(q, kv, sink, idx, out, B, M, H, N, K, scale, ws, stream);
    default: return launch_mla_nw<4>(q, kv, sink, idx, out, B, M, H, N, K, scale, ws, stream);
  }
}

// ---------------------------------------------------------------------------------------------------------
// Small kv sets (N <= 64 keys per batch, Dqk = Dv = 128): the dense count-mask form.  A batch's whole kv fits in
// LDS, so it is staged once per workgroup and every query scores all N keys densely on the MFMA; the top-k list
// only says how often each key counts.  Per query and wave (16 heads): the key counts (LDS atomics over the index
// list: invalid indices count nowhere, duplicates with multiplicity), S^T = K Q^T for all keys, the softmax over
// the counted keys with the sink, p = count * exp2(s - m), and O^T = V^T P^T, whose output layout gives each lane
// four consecutive columns of one head, staged through LDS into contiguous 16-byte stores.  Each workgroup covers
// a contiguous range of one batch's query groups (so its staged kv never changes), and each wave loads the next
// query's q rows and indices before computing the current one.  This replaces the gather kernel where each
// query's work is one short chunk and the launch is bound by q and output traffic.
constexpr int kDenseMaxN = 64;
constexpr int kDenseMaxK = 256;
constexpr int kDenseOutRow = 136;  // bf16 elements per staged output row (128 + 8 of padding)
// queries in flight per wave beyond the one computed: 1 keeps the kernel at 124 VGPRs, four waves per SIMD
// (139.8 us at the drop-in shape; 2 and 3 prefetched: 141.3 and 144.5 us at three waves per SIMD)
constexpr int kDensePrefetch = 1;

template <int NC, int KPL, int PD>  // 32-key chunks: N <= 32 NC; indices per lane: K <= 64 KPL; queries prefetched
__global__ __launch_bounds__(256) void sparse_attn_dense_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ kv, const float *__restrict__ sink,
    const int32_t *__restrict__ idx, uint16_t *__restrict__ out, int64_t M, int H, int N, int K, int GW, int64_t gpb,
    int64_t per_wg, int64_t rpb, float scale_log2) {
  using Sh = SaShape<128, 128, 1>;
  constexpr int D = 128, UPR = 16, NT = 2 * NC, CT = 8;
  constexpr int KEYS = 32 * NC;
  __shared__ __attribute__((aligned(16))) uint16_t kvs[KEYS * D];
  __shared__ __attribute__((aligned(16))) uint32_t cnt[4][KEYS];
  __shared__ __attribute__((aligned(16))) uint16_t ost[4][16 * kDenseOutRow];  // each wave's output rows
  const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qpi = 4 / GW;                          // queries per group
  const int qsub = wave / GW, head = 16 * (wave % GW) + l16;
  // the workgroup's range: groups [g0, g1) of batch bcur (rpb ranges of per_wg groups per batch), so the staged kv
  // rows never change during the loop
  const int64_t bcur = blockIdx.x / rpb;
  const int64_t g0 = bcur * gpb + (blockIdx.x % rpb) * per_wg;
  const int64_t g1 = g0 + per_wg < (bcur + 1) * gpb ? g0 + per_wg : (bcur + 1) * gpb;
  if (g0 >= g1) return;  // uniform per workgroup

  // the batch's kv rows into LDS (swizzled like the gather kernel's chunks); rows N .. KEYS - 1 are zero
  auto stage = [&](int64_t b) {
    const uint4 *src = reinterpret_cast<const uint4 *>(kv + b * N * D);
#pragma unroll
    for (int i = 0; i < KEYS * UPR / 256; ++i) {
      const int u = tid + 256 * i, key = u / UPR, un = u % UPR;
      const uint4 v = key < N ? src[key * UPR + un] : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4 *>(kvs + Sh::slot(key, 0, un) * 8) = v;
    }
  };
  // the wave's query row in the batch for group gq; row >= M for the idle waves of a batch's last group
  auto query_row = [&](int64_t gq) { return (gq - bcur * gpb) * qpi + qsub; };
  // q B-fragments Q[head][32j + 8g .. +7] and this lane's indices (lane + 64 i): every load unconditional, from a
  // clamped address (a load behind a branch makes the compiler wait for all loads where the paths join, which
  // would drain the prefetch); indices past K are masked where they are used (a select on a loaded value here
  // would wait for the load)
  auto load = [&](int64_t gq, uint4 (&qf)[4], int32_t (&ix)[KPL]) {
    const int64_t m = query_row(gq);
    const int64_t qm = bcur * M + (m < M ? m : M - 1);
    const uint16_t *qrow = q + (qm * H + head) * D + 8 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j) qf[j] = *reinterpret_cast<const uint4 *>(qrow + 32 * j);
    const int32_t *irow = idx + qm * K;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int t = lane + 64 * i;
      ix[i] = irow[t < K ? t : K - 1];
    }
  };

  // per-lane LDS element offsets: QK key 16t + l16, unit 4j + g; PV (transpose reads) keys 4g + (l16 >> 2) (+16),
  // unit 2cc + ((l16 & 3) >> 1), 8-byte half l16 & 1 (the gather kernel's layout)
  int qk0[4], pv0[CT];
#pragma unroll
  for (int j = 0; j < 4; ++j) qk0[j] = Sh::slot(l16, 0, 4 * j + g) * 8;
#pragma unroll
  for (int cc = 0; cc < CT; ++cc)
    pv0[cc] = Sh::slot(4 * g + (l16 >> 2), 0, 2 * cc + ((l16 & 3) >> 1)) * 8 + 4 * (l16 & 1);
  const float skl = sink[head] * kLog2e;

  // a ring of PD + 1 queries' q rows and indices in registers: the step computing query gq (slot s) first loads
  // query gq + PD into the slot that query gq - 1 used.  The loop is unrolled over the ring, so every slot is a
  // fixed set of registers: moving a value whose load is in flight would make the wave wait for it.
  stage(bcur);
  uint4 qr[PD + 1][4];
  int32_t ir[PD + 1][KPL];
#pragma unroll
  for (int d = 0; d < PD; ++d) load(g0 + d < g1 ? g0 + d : g1 - 1, qr[d], ir[d]);
  __syncthreads();
  uint32_t *cw = cnt[wave];
  auto compute = [&](int64_t gq, const uint4 (&qf)[4], const int32_t (&ix)[KPL]) {
    const int64_t m = query_row(gq);
    // idle waves (m >= M: past the batch's last row) compute row M - 1 and store nothing: the compute is not
    // behind a branch, where the compiler would wait for every prefetched load at the join
    {
      const int64_t qm = bcur * M + (m < M ? m : M - 1);
      // key counts of this query (the wave's own copy)
      if (lane < KEYS) cw[lane] = 0u;
#pragma unroll
      for (int i = 0; i < KPL; ++i)
        if (lane + 64 * i < K && ix[i] >= 0 && ix[i] < N) atomicAdd(&cw[ix[i]], 1u);
      uint4 c4[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) c4[t] = *reinterpret_cast<const uint4 *>(&cw[16 * t + 4 * g]);
      // S^T = K Q^T: lane holds keys 16t + 4g + r of head l16
      f32x4_t st[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        st[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          st[t] = mfma16(*reinterpret_cast<const uint4 *>(kvs + qk0[j] + 16 * t * UPR * 8), qf[j], st[t]);
      }
      // softmax over the counted keys and the sink
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t cv[4] = {c4[t].x, c4[t].y, c4[t].z, c4[t].w};
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (cv[r] != 0u) mx = fmaxf(mx, st[t][r] * scale_log2);
      }
      mx = fmaxf(rows_max(mx), skl);
      float p[NT][4], psum = 0.f;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t cv[4] = {c4[t].x, c4[t].y, c4[t].z, c4[t].w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[t][r] = (cv[r] != 0u && mx != -INFINITY)
                        ? static_cast<float>(cv[r]) * fast_exp2(st[t][r] * scale_log2 - mx) : 0.f;
          psum += p[t][r];
        }
      }
      const float den = rows_sum(psum) + (mx == -INFINITY ? 0.f : fast_exp2(skl - mx));
      const float inv = den > 0.f ? 1.f / den : 0.f;
      // O^T = V^T P^T: P^T is the B operand in the key order of the gather kernel's PV (keys 4g + r, 16 + 4g + r
      // of each 32-key chunk), V^T its V fragments as the A operand
      f32x4_t ot[CT];
#pragma unroll
      for (int cc = 0; cc < CT; ++cc) ot[cc] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 pb = make_uint4(pack_bf16x2(p[2 * c][0], p[2 * c][1]), pack_bf16x2(p[2 * c][2], p[2 * c][3]),
                                    pack_bf16x2(p[2 * c + 1][0], p[2 * c + 1][1]),
                                    pack_bf16x2(p[2 * c + 1][2], p[2 * c + 1][3]));
        const uint16_t *kc = kvs + c * 32 * UPR * 8;
#pragma unroll
        for (int cc = 0; cc < CT; ++cc) {
          const uint2 b0 = lds_read_tr16(kc + pv0[cc]);
          const uint2 b1 = lds_read_tr16(kc + pv0[cc] + 16 * UPR * 8);
          ot[cc] = mfma16(make_uint4(b0.x, b0.y, b1.x, b1.y), pb, ot[cc]);
        }
      }
      // lane: O[head l16][16cc + 4g .. + 3].  The wave's 16 output rows (4 KiB, contiguous in out) go through LDS
      // (rows padded to 272 bytes: no bank conflicts) and leave as 1 KiB runs of 16-byte stores; storing the lanes'
      // 8-byte pieces directly writes 32 bytes into each of 16 rows per instruction, 23% slower at the drop-in shape.
      // Unconditional: an idle wave computes row M - 1 with the same head block as the wave that owns that row, so
      // it writes the same bytes to the same place (a store behind a branch would make the compiler's wait for the
      // next prefetched rows also wait for these stores to complete).
      uint16_t *ob = ost[wave];
#pragma unroll
      for (int cc = 0; cc < CT; ++cc)
        *reinterpret_cast<uint2 *>(ob + l16 * kDenseOutRow + 16 * cc + 4 * g) =
            make_uint2(pack_bf16x2(ot[cc][0] * inv, ot[cc][1] * inv), pack_bf16x2(ot[cc][2] * inv, ot[cc][3] * inv));
      uint4 *odst = reinterpret_cast<uint4 *>(out + (qm * H + 16 * (wave % GW)) * D);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = lane + 64 * i;  // 16-byte chunk c of the wave's 4 KiB: row c / 16, chunk c % 16
        odst[c] = *reinterpret_cast<const uint4 *>(ob + (c >> 4) * kDenseOutRow + 8 * (c & 15));
      }
    }
  };
  for (int64_t gb = g0; gb < g1; gb += PD + 1) {
#pragma unroll
    for (int sl = 0; sl <= PD; ++sl) {
      const int64_t gq = gb + sl;
      if (gq >= g1) break;  // uniform per workgroup
      load(gq + PD < g1 ? gq + PD : g1 - 1, qr[(sl + PD) % (PD + 1)], ir[(sl + PD) % (PD + 1)]);
      compute(gq, qr[sl], ir[sl]);
    }
  }
}

inline bool use_dense(int64_t Dqk, int64_t Dv, int64_t H, int64_t N, int64_t K, const void *out) {
  static_assert(kDenseMaxK == 256, "the launcher instantiates 1 and 4 indices per lane");
  return Dqk == 128 && Dv == 128 && N <= kDenseMaxN && K <= kDenseMaxK && (H == 16 || H == 32 || H == 64) &&
         aligned(out, 16);
}

int launch_sa_dense(const uint16_t *q, const uint16_t *kv, const float *sink, const int32_t *idx, uint16_t *out,
                    int64_t B, int64_t M, int64_t H, int64_t N, int64_t K, float scale, hipStream_t stream) {
  const int gw = static_cast<int>(H / 16);  // waves per query: 1, 2 or 4
  const int64_t qpi = 4 / gw;
  const int64_t gpb = ceil_div(M, qpi);     // query groups per batch
  int dev = 0, cus = 0;
  KS_CHECK_HIP(hipGetDevice(&dev));
  KS_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const float sl2 = scale * kLog2e;
  const int h32 = static_cast<int>(H), n32 = static_cast<int>(N), k32 = static_cast<int>(K);
  // about as many workgroups as fit at once (the kernel's occupancy), each over a contiguous range of one batch's
  // query groups: rpb ranges of `per` groups per batch
  auto run = [&](auto kern) -> int {
    int per_cu = 0;
    KS_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, 0));
    const int64_t target = static_cast<int64_t>(cus > 0 ? cus : 1) * (per_cu > 0 ? per_cu : 1);
    const int64_t want_rpb = ceil_div(target, B) < gpb ? ceil_div(target, B) : gpb;
    const int64_t per = ceil_div(gpb, want_rpb);
    const int64_t rpb = ceil_div(gpb, per);
    const int64_t wgs = B * rpb;
    KS_CHECK_ARG(wgs < (int64_t(1) << 31), "sparse attention (dense): %lld workgroups", (long long)wgs);
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(wgs)), dim3(256), 0, stream, q, kv, sink, idx, out, M, h32,
                       n32, k32, gw, gpb, per, rpb, sl2);
    KS_CHECK_LAUNCH("sparse_attn_dense_kernel");
    return KS_OK;
  };
  constexpr int PD = kDensePrefetch;
  if (N <= 32 && K <= 64) return run(sparse_attn_dense_kernel<1, 1, PD>);
  if (N <= 32) return run(sparse_attn_dense_kernel<1, 4, PD>);
  if (K <= 64) return run(sparse_attn_dense_kernel<2, 1, PD>);
  return run(sparse_attn_dense_kernel<2, 4, PD>);
}

// ---------------------------------------------------------------------------------------------------------
// Dense top-k lists over larger kv sets (Dqk = Dv = 128, K >= N / 4): the count-mask form over key splits.  At
// 25% density the gather kernel spends each 32-key chunk on one query's 16 heads, a short chain of dependent
// QK -> softmax -> PV with ~16 MFMAs, and gathers every row for every query.  Here every query scores every key of
// its split on the MFMA, and the top-k list only says how often each key counts (the reference's dense design,
// optimized/sparse_attention/design.md:46-69, there for N = 32).  That is 4x the MFMA work at 25% density, done
// as long streams of 32 x 32 x 16 MFMAs on key chunks shared by the workgroup's waves.
//   workgroup  128 consecutive (query, head) rows of one batch (4 waves x 32 rows; H divides 128) x one key split
//              of KR keys; one wave per SIMD (registers: 4 x 16 O^T accumulators, 8 q fragments, two S^T tiles)
//   counts     the workgroup's index rows read once (all loads in flight together) and counted into LDS with
//              ds_add: invalid indices count nowhere, duplicates with multiplicity
//   chunks     32 keys x 128 dims, DMA'd into a 4-buffer ring in a swizzled row-major layout; at chunk c
//              chunk c + 1 has landed and chunks c + 2, c + 3 are in flight (one barrier per chunk)
//   QK^T       S^T = K Q^T (M = 32 keys, N = 32 rows, K = 16 dims); lane (row l%32, half h = l/32) receives keys
//              8j + 4h + r (j, r = 0..3).  Chunk c + 1's QK is issued before chunk c's softmax.
//   softmax    p = 2^(s + log2(count) - m) with the lazily updated reference max of the gather kernel (the counts
//              become log2 weights in LDS, -inf for keys counted nowhere); a row's keys are split over lanes l and
//              l ^ 32, which share the max through v_permlane32_swap
//   PV         O^T = V^T P^T (M = 32 dv, N = 32 rows, K = 16 keys): the k order of a step is the lane's own key
//              order (keys 16s + 4h + e, then 16s + 8 + 4h + e), so P^T is the lane's probabilities as they
//              are, and the matching V^T fragment is two ds_read_b64_tr_b16 reads.  O^T keeps one row per lane,
//              so a rescale needs no exchange.
// Partial ranges (O in bf16, max, sum) go through sparse_attn_combine_kernel; one split finalises in place.
// Measured slower than the gather kernel at every density tried (config 3: 27 against 15 us; at 100% density 19
// against 15 us), so ks_sparse_attn does not dispatch to it; ks_dbg_sparse_attn_count exposes it for timing.
constexpr int kCntRows = 128;       // (query, head) rows per workgroup
constexpr int kCntMaxKR = 2048;     // keys per split (LDS counts: 128 / H queries x KR x 4 bytes)
constexpr int kCntBufs = 4;         // chunk ring: chunks c + 1 and c + 2 in flight while chunk c is computed
constexpr int kCntTargetWgs = 256;  // one workgroup per CU
constexpr int kCntIdxBatch = 16;    // index loads in flight per thread while counting

typedef float f32x16_t __attribute__((ext_vector_type(16)));
__device__ __forceinline__ f32x16_t mfma32(uint4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                  0, 0, 0);
}

__global__ __launch_bounds__(256, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) void sparse_attn_count_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ kv, const float *__restrict__ sink,
    const int32_t *__restrict__ idx, uint16_t *__restrict__ out, uint16_t *__restrict__ part_o,
    float *__restrict__ part_ml, int64_t M, int H, int N, int K, int NS, int KR, int64_t tgb, float scale_log2,
    int idx_vec) {
  constexpr int D = 128, BUF = 32 * D;            // bf16 elements per chunk buffer
  extern __shared__ uint4 smem_cnt[];
  uint16_t *kb = reinterpret_cast<uint16_t *>(smem_cnt);               // [kCntBufs][BUF]
  uint32_t *cnt = reinterpret_cast<uint32_t *>(kb + kCntBufs * BUF);   // [128 / H][KR]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c32 = lane & 31, h2 = lane >> 5;
  // the splits of one row block are dealt to one XCD (workgroup i runs on XCD i mod 8): they share its index rows
  const int64_t nblk = gridDim.x;
  const int64_t lb = (nblk % 8 == 0) ? (blockIdx.x % 8) * (nblk / 8) + blockIdx.x / 8 : blockIdx.x;
  const int s = static_cast<int>(lb % NS);
  const int64_t tg = (lb / NS) % tgb;
  const int64_t b = lb / (static_cast<int64_t>(NS) * tgb);
  const int64_t MH = M * H;
  const int64_t row0 = tg * kCntRows;  // the workgroup's first row of batch b (a multiple of H)
  const int QW = kCntRows / H;
  const int64_t m0 = row0 / H;
  const int qv = static_cast<int>(M - m0 < QW ? M - m0 : QW);  // queries of the workgroup inside the batch
  const int k_lo = s * KR, k_hi = k_lo + KR < N ? k_lo + KR : N;
  const int nch = (k_hi - k_lo + 31) / 32;  // >= 1: the host plan leaves no split empty
  const global_ptr<const uint16_t> kvb = uniform_ptr(kv + b * static_cast<int64_t>(N) * D);
  const uint32_t kb_lds = __builtin_amdgcn_readfirstlane(lds_addr(kb));

  // ---- chunk layout: unit u of key k in slot 16 k + (u ^ swz(k)), swz(k) = 4 (k & 3) + 2 ((k >> 2) & 1).  The QK
  // reads (8 keys, one unit) and the PV transpose reads (per 32 lanes 4 keys x 4 units, or 4 units + 2 for keys
  // 4..7 of an 8-key group) then hit distinct banks.  DMA slot 64 (wave + 4 i) + lane holds unit (slot % 16) ^
  // swz(key) of key slot / 16.
  auto swz = [](int k) { return 4 * (k & 3) + 2 * ((k >> 2) & 1); };
  auto cslot = [&](int k, int u) { return 16 * k + (u ^ swz(k)); };
  int dkey[2], doff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int sl = 64 * (wave + 4 * i) + lane;
    dkey[i] = sl / 16;
    doff[i] = ((sl % 16) ^ swz(dkey[i])) * 16;
  }
  auto dma_chunk = [&](int c, int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int key = k_lo + 32 * c + dkey[i];
      key = key < N ? key : N - 1;  // past the split's end: a real row, counted nowhere
      dma16((const void *)kvb, static_cast<uint32_t>(key) * (D * 2) + doff[i],
            kb_lds + (buf * BUF + 64 * (wave + 4 * i) * 8) * 2);
    }
  };
#pragma unroll
  for (int i = 0; i < kCntBufs - 1; ++i)
    if (i < nch) dma_chunk(i, i);

  // ---- q B-fragments: row (wave's 32 rows, lane c32), dims 16j + 8h .. +7; rows past the batch read its last row
  const int64_t qrow = row0 + 32 * wave + c32;
  const bool row_ok = qrow < MH;
  const uint16_t *qp = q + (b * MH + (row_ok ? qrow : MH - 1)) * D + 8 * h2;
  uint4 qf[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) qf[j] = *reinterpret_cast<const uint4 *>(qp + 16 * j);

  // ---- key counts of the workgroup's queries over [k_lo, k_hi)
  for (int i = tid * 4; i < QW * KR; i += 1024) *reinterpret_cast<uint4 *>(cnt + i) = make_uint4(0, 0, 0, 0);
  __syncthreads();
  {
    const int32_t *ib = idx + (b * M + m0) * static_cast<int64_t>(K);  // qv consecutive index rows
    // row of element e of the qv x K index block (the float quotient is within one of e / K: qv <= 8)
    const float inv_k = 1.f / static_cast<float>(K);
    auto row_of = [&](int e) {
      int r = static_cast<int>(static_cast<float>(e) * inv_k);
      r -= static_cast<int64_t>(r) * K > e ? 1 : 0;
      r += static_cast<int64_t>(r + 1) * K <= e ? 1 : 0;
      return r;
    };
    const uint32_t span = static_cast<uint32_t>(k_hi - k_lo);
    auto count = [&](int rbase, int32_t v) {  // rbase = row * KR - k_lo
      if (static_cast<uint32_t>(v - k_lo) < span) atomicAdd(&cnt[rbase + v], 1u);
    };
    const int tot = qv * K;
    if (idx_vec) {  // K % 4 == 0 and 16-byte aligned rows: the four indices of an int4 share a row
      const int4 *ib4 = reinterpret_cast<const int4 *>(ib);
      const int n4 = tot >> 2;
      for (int base = 0; base < n4; base += 256 * kCntIdxBatch) {
        int4 v[kCntIdxBatch];
#pragma unroll
        for (int j = 0; j < kCntIdxBatch; ++j) {
          const int u = base + 256 * j + tid;
          v[j] = ib4[u < n4 ? u : n4 - 1];
        }
#pragma unroll
        for (int j = 0; j < kCntIdxBatch; ++j) {
          const int u = base + 256 * j + tid;
          if (u < n4) {
            const int rb = row_of(4 * u) * KR - k_lo;
            count(rb, v[j].x);
            count(rb, v[j].y);
            count(rb, v[j].z);
            count(rb, v[j].w);
          }
        }
      }
    } else {
      for (int base = 0; base < tot; base += 256 * kCntIdxBatch) {
        int32_t v[kCntIdxBatch];
#pragma unroll
        for (int j = 0; j < kCntIdxBatch; ++j) {
          const int e = base + 256 * j + tid;
          v[j] = ib[e < tot ? e : tot - 1];
        }
#pragma unroll
        for (int j = 0; j < kCntIdxBatch; ++j) {
          const int e = base + 256 * j + tid;
          if (e < tot) count(row_of(e) * KR - k_lo, v[j]);
        }
      }
    }
  }
  __syncthreads();
  // counts -> log2 weights: p = 2^(s + log2(count) - m); -inf for keys counted nowhere
  for (int i = tid * 4; i < QW * KR; i += 1024) {
    uint4 *w = reinterpret_cast<uint4 *>(cnt + i);
    const uint4 c = *w;
    auto lw = [](uint32_t n) { return __float_as_uint(n == 0u ? -INFINITY : __log2f(static_cast<float>(n))); };
    *w = make_uint4(lw(c.x), lw(c.y), lw(c.z), lw(c.w));
  }
  wait_dma();
  __syncthreads();  // weights complete, chunks 0 to 2 visible

  // ---- per-lane LDS element offsets.  QK: key c32, unit 2j + h (swizzled per j).  PV (transpose reads): lane
  // 16R + 4e + jj addresses key 4(R >> 1) + e (+ 8, + 16 s), columns 32 ct + 16 (R & 1) + 4 jj .. +3
  int qk_off[8], pv_off[4];
#pragma unroll
  for (int j = 0; j < 8; ++j) qk_off[j] = cslot(c32, 2 * j + h2) * 8;
  {
    const int R = lane >> 4, e = (lane >> 2) & 3, jj = lane & 3;
    const int key = 4 * (R >> 1) + e;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) pv_off[ct] = cslot(key, 4 * ct + 2 * (R & 1) + (jj >> 1)) * 8 + 4 * (jj & 1);
  }
  const int qi = (32 * wave + c32) / H;  // the lane's query in the workgroup's count rows
  const float *crow = reinterpret_cast<const float *>(cnt) + qi * KR + 4 * h2;  // log2 weights

  // LDS reads of a chunk: the lane's 8 K fragments, its 4 x 2 V^T fragments (two transpose reads each) and the
  // log2 weights of its 16 keys
  auto kfrags = [&](int buf, uint4(&kf)[8]) {
    const uint16_t *kbp = kb + buf * BUF;
#pragma unroll
    for (int j = 0; j < 8; ++j) kf[j] = *reinterpret_cast<const uint4 *>(kbp + qk_off[j]);
  };
  auto vfrags = [&](int buf, uint4(&vf)[4][2]) {
    const uint16_t *kbp = kb + buf * BUF;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const uint2 v0 = lds_read_tr16(kbp + pv_off[ct] + (16 * s2) * 16 * 8);
        const uint2 v1 = lds_read_tr16(kbp + pv_off[ct] + (16 * s2 + 8) * 16 * 8);
        vf[ct][s2] = make_uint4(v0.x, v0.y, v1.x, v1.y);
      }
  };
  auto weights = [&](int c, float (&w)[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 v = *reinterpret_cast<const float4 *>(crow + 32 * c + 8 * j);
      w[4 * j] = v.x, w[4 * j + 1] = v.y, w[4 * j + 2] = v.z, w[4 * j + 3] = v.w;
    }
  };
  // t = s + log2(weight) and its row max over the chunk (lanes l and l ^ 32 hold the row's two key halves)
  auto scores = [&](const f32x16_t &sc, const float (&w)[16], float (&t)[16]) {
    float cmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      t[i] = fmaf(sc[i], scale_log2, w[i]);
      cmax = fmaxf(cmax, t[i]);
    }
    float a = cmax, bb = cmax;
    swap32(a, bb);
    return fmaxf(a, bb);
  };

  float m_ref = -INFINITY, l_run = 0.f;  // per row (lanes l and l ^ 32 hold the same values)
  f32x16_t o[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) o[ct] = f32x16_t{};
  // u: the current chunk's exponents t - m_ref (-inf for keys counted nowhere)
  float u[16];
  {
    uint4 kf[8];
    float w[16], t[16];
    kfrags(0, kf);
    weights(0, w);
    f32x16_t sc = {};
#pragma unroll
    for (int j = 0; j < 8; ++j) sc = mfma32(kf[j], qf[j], sc);
    m_ref = scores(sc, w, t);
    const float m_use = m_ref == -INFINITY ? 0.f : m_ref;  // no counted key: every t is -inf, p = 0
#pragma unroll
    for (int i = 0; i < 16; ++i) u[i] = t[i] - m_use;
  }

  // Two stages per chunk c: (A) chunk c + 1's QK MFMAs beside chunk c's exponentials and bf16 packing, (B) chunk
  // c's PV MFMAs beside chunk c + 1's scores and row max.  A rescale for chunk c + 1 (rare) then scales O, which
  // holds chunk c, and the sum.  On the last chunk the "next" buffer and weights are stale and unused.
  static_assert(kCntBufs == 4, "the waits below keep one chunk (two DMA instructions per thread) in flight");
  for (int c = 0; c < nch; ++c) {
    if (c + 2 < nch) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");  // this thread's part of chunk c + 1
    else if (c + 1 < nch) wait_dma();
    __syncthreads();  // chunk c + 1 visible; every wave is done with chunk c - 1's buffer
    if (c + 3 < nch) dma_chunk(c + 3, (c + 3) % kCntBufs);
    uint4 kf[8], vf[4][2];
    float w[16];
    kfrags((c + 1) % kCntBufs, kf);
    vfrags(c % kCntBufs, vf);
    weights(c + 1 < nch ? c + 1 : c, w);
    // (A)
    f32x16_t sn = {};
#pragma unroll
    for (int j = 0; j < 8; ++j) sn = mfma32(kf[j], qf[j], sn);
    float p[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      p[i] = fast_exp2(u[i]);
      l_run += p[i];
    }
    uint4 pb[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
      pb[s2] = make_uint4(pack_bf16x2(p[8 * s2], p[8 * s2 + 1]), pack_bf16x2(p[8 * s2 + 2], p[8 * s2 + 3]),
                          pack_bf16x2(p[8 * s2 + 4], p[8 * s2 + 5]), pack_bf16x2(p[8 * s2 + 6], p[8 * s2 + 7]));
    // (B)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) o[ct] = mfma32(vf[ct][s2], pb[s2], o[ct]);
    float t[16];
    const float cmax = scores(sn, w, t);
    const float m_use = m_ref == -INFINITY ? 0.f : m_ref;
#pragma unroll
    for (int i = 0; i < 16; ++i) u[i] = t[i] - m_use;
    const bool need = cmax > m_ref + kRescaleTau;  // false for cmax = -inf; true for a first counted chunk
    if (c + 1 < nch && __builtin_amdgcn_ballot_w64(need) != 0ull) {
      const float m_new = need ? cmax : m_ref;
      const float alpha = need ? (m_ref == -INFINITY ? 0.f : fast_exp2(m_ref - m_new)) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) o[ct] *= alpha;
      m_ref = m_new;
      const float m_use2 = m_ref == -INFINITY ? 0.f : m_ref;
#pragma unroll
      for (int i = 0; i < 16; ++i) u[i] = t[i] - m_use2;
    }
  }

  // ---- finalise: lane holds row qrow, dv columns 32 ct + 8 (i / 4) + 4h + i % 4
  {
    float a = l_run, bb = l_run;
    swap32(a, bb);
    l_run = a + bb;
  }
  if (!row_ok) return;
  const int64_t m = qrow / H;
  const int h = static_cast<int>(qrow % H);
  const int64_t qm = b * M + m;
  if (NS == 1) {
    const float sk = sink[h] * kLog2e;
    const float z = fmaxf(m_ref, sk);
    float so = 0.f;
    if (z != -INFINITY) {
      const float e = m_ref == -INFINITY ? 0.f : exp2f(m_ref - z);
      const float den = l_run * e + exp2f(sk - z);
      so = den > 0.f ? e / den : 0.f;
    }
    uint16_t *orow = out + (qm * H + h) * D + 4 * h2;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        *reinterpret_cast<uint2 *>(orow + 32 * ct + 8 * jj) =
            make_uint2(pack_bf16x2(o[ct][4 * jj] * so, o[ct][4 * jj + 1] * so),
                       pack_bf16x2(o[ct][4 * jj + 2] * so, o[ct][4 * jj + 3] * so));
  } else {
    const int64_t pr = (qm * NS + s) * H + h;
    uint16_t *po = part_o + pr * D + 4 * h2;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        *reinterpret_cast<uint2 *>(po + 32 * ct + 8 * jj) = make_uint2(pack_bf16x2(o[ct][4 * jj], o[ct][4 * jj + 1]),
                                                                       pack_bf16x2(o[ct][4 * jj + 2], o[ct][4 * jj + 3]));
    if (h2 == 0) {
      part_ml[pr * 2] = m_ref;
      part_ml[pr * 2 + 1] = l_run;
    }
  }
}

constexpr size_t kCntMaxShmem = 64 * 1024;  // dynamic LDS without a per-kernel attribute
inline size_t count_shmem(int64_t H, int64_t kr) {
  return static_cast<size_t>(kCntBufs) * 32 * 128 * 2 + static_cast<size_t>(kCntRows / H) * kr * 4;
}

struct CntPlan {
  int ns, kr;
  int64_t tgb;  // row blocks per batch
};

// The count-mask kernel takes dense lists (K >= N / 4) over kv sets past the small-kv kernel's, with whole
// 128-row blocks (M H >= 128, H dividing 128).  Splits: about one workgroup per CU, at most kCntMaxKR keys each,
// and no more ranges than the gather plan's, whose workspace size the caller was given (the workspace query does
// not see N).
inline bool count_plan(int64_t B, int64_t M, int64_t H, int64_t N, int64_t K, const void *out, CntPlan &p) {
  if (N <= kDenseMaxN || K * 4 < N || kCntRows % H != 0 || M * H < kCntRows || !aligned(out, 8)) return false;
  if (K * (kCntRows / H) >= (int64_t(1) << 31)) return false;  // the workgroup's index block is int-indexed
  const int64_t tgb = ceil_div(M * H, kCntRows);
  int64_t ns = ceil_div(kCntTargetWgs, B * tgb);
  const int64_t ns_min = ceil_div(N, kCntMaxKR);
  const int64_t ns_max = ceil_div(N, 4 * 32) > ns_min ? ceil_div(N, 4 * 32) : ns_min;  // >= 4 chunks per split
  ns = ns < ns_min ? ns_min : ns > ns_max ? ns_max : ns;
  const SaSplit sp = split_plan(B, M, H, K);
  if (ns > sp.ns) ns = sp.ns;
  if (ns < ns_min) return false;
  const int64_t kr = ceil_div(ceil_div(N, ns), 32) * 32;
  ns = ceil_div(N, kr);  // no empty split (and no more than before)
  if (count_shmem(H, kr) > kCntMaxShmem) return false;
  if (B * tgb * ns >= (int64_t(1) << 31)) return false;
  p = CntPlan{static_cast<int>(ns), static_cast<int>(kr), tgb};
  return true;
}

int launch_sa_count(const CntPlan &p, const uint16_t *q, const uint16_t *kv, const float *sink, const int32_t *idx,
                    uint16_t *out, int64_t B, int64_t M, int64_t H, int64_t N, int64_t K, float scale, void *ws,
                    hipStream_t stream) {
  float *part_ml = nullptr;
  uint16_t *part_o = nullptr;
  if (p.ns > 1) {
    part_ml = static_cast<float *>(ws);
    part_o = reinterpret_cast<uint16_t *>(part_ml + B * M * p.ns * H * 2);
  }
  const size_t shmem = count_shmem(H, p.kr);
  const int idx_vec = (K % 4 == 0 && aligned(idx, 16)) ? 1 : 0;
  const int64_t wgs = B * p.tgb * p.ns;
  hipLaunchKernelGGL(sparse_attn_count_kernel, dim3(static_cast<unsigned>(wgs)), dim3(256), shmem, stream, q, kv, sink,
                     idx, out, part_o, part_ml, M, static_cast<int>(H), static_cast<int>(N), static_cast<int>(K), p.ns,
                     p.kr, p.tgb, scale * kLog2e, idx_vec);
  KS_CHECK_LAUNCH("sparse_attn_count_kernel");
  if (p.ns > 1) {
    const int64_t rows = B * M * H;
    const int rc = launch_combine<128>(part_o, part_ml, sink, out, rows, static_cast<int>(H), p.ns, stream);
    if (rc != KS_OK) return rc;
  }
  return KS_OK;
}

template <int DQK, int DV>
int launch_sa(const uint16_t *q, const uint16_t *kv, const float *sink, const int32_t *idx, uint16_t *out,
              int64_t B, int64_t M, int64_t H, int64_t N, int64_t K, float scale, void *ws, hipStream_t stream) {
  switch (waves_per_group(H)) {
    case 1: return launch_sa_gw<DQK, DV, 1>(q, kv, sink, idx, out, B, M, H, N, K, scale, ws, stream);
    case 2: return launch_sa_gw<DQK, DV, 2>(q, kv, sink, idx, out, B, M, H, N, K, scale, ws, stream);
    case 4: return launch_sa_gw<DQK, DV, 4>(q, kv, sink, idx, out, B, M, H, N, K, scale, ws, stream);
    default: return launch_sa_gw<DQK, DV, 8>(q, kv, sink, idx, out, B, M, H, N, K, scale, ws, stream);
  }
}

size_t sa_workspace(int64_t B, int64_t M, int64_t H, int64_t DQK, int64_t K, int64_t DV) {
  const SaSplit sp = use_mla(DQK, DV, H, K) ? mla_plan(B, M, K) : split_plan(B, M, H, K);
  if (sp.ns <= 1) return 0;
  return static_cast<size_t>(B * M * sp.ns * H) * (2 * sizeof(float) + DV * sizeof(uint16_t));
}

}  // namespace
}  // namespace ks

extern "C" size_t ks_sparse_attn_workspace_size(int64_t B, int64_t M, int64_t H, int64_t Dqk, int64_t Dv, int64_t K) {
  if (B <= 0 || M <= 0 || H <= 0 || K <= 0 || Dv <= 0) return 0;
  return ks::sa_workspace(B, M, H, Dqk, K, Dv);
}

extern "C" int ks_sparse_attn(const uint16_t *q, const uint16_t *kv, const float *sink, const int32_t *idx,
                              uint16_t *out, int64_t B, int64_t M, int64_t H, int64_t Dqk, int64_t Dv, int64_t N,
                              int64_t K, float scale, void *workspace, size_t workspace_bytes, void *stream) {
  ks::last_error().clear();
  KS_CHECK_ARG(B >= 0 && M >= 0 && N >= 1 && K >= 1 && H >= 1, "ks_sparse_attn: bad sizes B=%lld M=%lld N=%lld K=%lld H=%lld",
               (long long)B, (long long)M, (long long)N, (long long)K, (long long)H);
  KS_CHECK_ARG(H % 16 == 0 && H <= 128, "ks_sparse_attn: H=%lld must be a multiple of 16, at most 128", (long long)H);
  const bool d128 = Dqk == 128 && Dv == 128;
  const bool d576 = Dqk == 576 && Dv == 512;
  KS_CHECK_ARG(d128 || d576, "ks_sparse_attn: (Dqk, Dv)=(%lld, %lld); supported: (128, 128), (576, 512)",
               (long long)Dqk, (long long)Dv);
  KS_CHECK_ARG(M < 65536 && B < 65536, "ks_sparse_attn: M and B must be < 65536");
  KS_CHECK_ARG(K < (int64_t(1) << 31) && N * Dqk * 2 < (int64_t(1) << 32),
               "ks_sparse_attn: K must be < 2^31 and one batch's kv (N*Dqk*2 bytes) < 4 GiB");
  if (B * M == 0) return KS_OK;
  KS_CHECK_ARG(q && kv && sink && idx && out, "ks_sparse_attn: null pointer");
  KS_CHECK_ARG(ks::aligned(q, 16) && ks::aligned(kv, 16), "ks_sparse_attn: q and kv must be 16-byte aligned");
  const size_t need = ks::sa_workspace(B, M, H, Dqk, K, Dv);
  KS_CHECK_ARG(need == 0 || (workspace != nullptr && workspace_bytes >= need),
               "ks_sparse_attn: workspace of %zu bytes required, %zu given", need, workspace_bytes);
  KS_CHECK_ARG(need == 0 || ks::aligned(workspace, 16), "ks_sparse_attn: workspace must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (ks::use_dense(Dqk, Dv, H, N, K, out)) return ks::launch_sa_dense(q, kv, sink, idx, out, B, M, H, N, K, scale, st);
  if (d128) return ks::launch_sa<128, 128>(q, kv, sink, idx, out, B, M, H, N, K, scale, workspace, st);
  if (ks::use_mla(Dqk, Dv, H, K)) return ks::launch_mla(q, kv, sink, idx, out, B, M, H, N, K, scale, workspace, st);
  return ks::launch_sa<576, 512>(q, kv, sink, idx, out, B, M, H, N, K, scale, workspace, st);
}

// Diagnostic export (not in include/kswift.h): ks_sparse_attn's contract on the count-mask kernel, for the shapes its
// plan takes (Dqk = Dv = 128, K >= N / 4, N > 64, H dividing 128, M H >= 128).  ks_sparse_attn does not dispatch to
// it: at every density measured it was slower than the gather kernel.  Kept to time the dense formulation beside
// the gather kernel and to keep its parity tested.
extern "C" int ks_dbg_sparse_attn_count(const uint16_t *q, const uint16_t *kv, const float *sink, const int32_t *idx,
                                        uint16_t *out, int64_t B, int64_t M, int64_t H, int64_t N, int64_t K,
                                        float scale, void *workspace, size_t workspace_bytes, void *stream) {
  ks::last_error().clear();
  KS_CHECK_ARG(B >= 1 && M >= 1 && N >= 1 && K >= 1 && H >= 1 && M < 65536 && B < 65536 && K < (int64_t(1) << 31) &&
                   N * 256 < (int64_t(1) << 32),
               "ks_dbg_sparse_attn_count: bad sizes");
  KS_CHECK_ARG(q && kv && sink && idx && out && ks::aligned(q, 16) && ks::aligned(kv, 16),
               "ks_dbg_sparse_attn_count: null or misaligned pointer");
  ks::CntPlan cp;
  KS_CHECK_ARG(ks::count_plan(B, M, H, N, K, out, cp), "ks_dbg_sparse_attn_count: shape outside the kernel's plan");
  const size_t need = ks::sa_workspace(B, M, H, 128, K, 128);
  KS_CHECK_ARG(need == 0 || (workspace != nullptr && workspace_bytes >= need && ks::aligned(workspace, 16)),
               "ks_dbg_sparse_attn_count: workspace of %zu bytes required", need);
  return ks::launch_sa_count(cp, q, kv, sink, idx, out, B, M, H, N, K, scale, workspace,
                             static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------- the entry point that allocates nothing
// Split partials of ks_sparse_attn_noalloc live in this file-scope device array instead of a caller
// workspace.  Each GPU the library runs on holds its own copy (the code object's data on that device) for
// the life of the process; host code never names the array in a launch or a copy (its name is a host-side
// stand-in), only the device address hipGetSymbolAddress returns for the stream's device, resolved once per
// device.  Every partial range is written by the attention kernels before the combine kernel reads it in
// the same call, so nothing needs clearing; calls that overlap on one GPU share the array and race.
namespace ks {
constexpr size_t kSaScratchBytes = size_t(64) << 20;
}
static __device__ __align__(256) unsigned char scratch[ks::kSaScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::array<void *, kMaxDevices> g_scratch_ptr{};

// The scratch address on the device of `st` (the current device for the null stream).
int scratch_for_stream(hipStream_t st, void **ptr) {
  int cur = 0;
  KS_CHECK_HIP(hipGetDevice(&cur));
  int dev = cur;
  if (st != nullptr) {
    hipDevice_t d = 0;
    KS_CHECK_HIP(hipStreamGetDevice(st, &d));
    dev = static_cast<int>(d);
  }
  KS_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "ks_sparse_attn_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur) KS_CHECK_HIP(hipSetDevice(dev));
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    KS_CHECK_HIP(e);
    KS_CHECK_ARG(p != nullptr, "ks_sparse_attn_noalloc: no scratch address on device %d", dev);
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return KS_OK;
}
}  // namespace

extern "C" size_t ks_sparse_attn_noalloc_max_scratch(void) { return ks::kSaScratchBytes; }

extern "C" int ks_sparse_attn_noalloc(const uint16_t *q, const uint16_t *kv, const float *sink, const int32_t *idx,
                                      uint16_t *out, int64_t B, int64_t M, int64_t H, int64_t Dqk, int64_t Dv,
                                      int64_t N, int64_t K, float scale, void *stream) {
  ks::last_error().clear();
  const size_t need = ks_sparse_attn_workspace_size(B, M, H, Dqk, Dv, K);
  KS_CHECK_ARG(need <= ks::kSaScratchBytes,
               "ks_sparse_attn_noalloc: this shape needs %zu bytes of split scratch, the maximum is %zu bytes "
               "(call ks_sparse_attn with a workspace instead)", need, ks::kSaScratchBytes);
  void *ws = nullptr;
  if (need > 0 && B * M > 0) {
    const int rc = scratch_for_stream(static_cast<hipStream_t>(stream), &ws);
    if (rc != KS_OK) return rc;
  }
  return ks_sparse_attn(q, kv, sink, idx, out, B, M, H, Dqk, Dv, N, K, scale, ws, need, stream);
}
