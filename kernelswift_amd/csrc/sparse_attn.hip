// Sparse attention over gathered top-k KV rows with an attention sink (gfx950).
//
// Semantics: sparse_attn_ref (baseline/sparse_attention.py:5-42); replaces the reference's kvT transpose +
// dense-N megakernel (optimized/sparse_attention/op_kernel/fused_sparse_attn_basic_kernel.asc:535-648,
// transpose_kv_kernel.asc:35-63), which only handled N = 32 keys, with a real gather.
//
// Decomposition: the K indices of query (b, m) are split into NS ranges; workgroup (range, m, b) has one
// wave per 16 heads and walks its range in chunks of 32 keys:
//   gather   the chunk's kv rows (16-byte loads, invalid indices -> zero rows) into LDS twice: row-major
//            K (rows padded by 16 bytes so 16 lanes reading 16 keys hit distinct banks) and a key-interleaved
//            V copy [key/8][d][key%8] whose 8-key runs are MFMA B-operand columns;
//   QK^T     S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (M = 16 keys, N = 16 heads), the wave's q rows held
//            as B-fragments in VGPRs; lane (head = l%16, g = l/16) receives keys 4g..4g+3 of each 16-key tile;
//   softmax  online (running max / sum per head, base-2 exponentials), invalid keys -> 0;
//   PV       O = P V with M = 16 heads, N = 16 dv columns, K = 32 keys: a lane's 8 probabilities
//            {4g..4g+3, 16+4g..16+4g+3} are its A-fragment as-is, and V is read with the same key
//            permutation (two 8-byte LDS reads), so P never goes through LDS.
// NS == 1 finalises in place (sink added, bf16 store); otherwise partial (O, max, sum) go to the
// workspace and a combine kernel merges ranges with the sink (log-sum-exp).
#include "common.h"

namespace ks {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kKC = 32;  // keys per chunk
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                  0, 0, 0);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16_rne(lo)) | (static_cast<uint32_t>(f32_to_bf16_rne(hi)) << 16);
}

// Split heuristic shared by the launcher and the workspace-size query: aim for ~2048 waves in flight.
__host__ __device__ inline int choose_splits(int64_t B, int64_t M, int64_t H, int64_t K) {
  const int64_t waves_per_query = (H + 15) / 16;
  const int64_t chunks = (K + kKC - 1) / kKC;
  int64_t ns = 2048 / (B * M * waves_per_query > 0 ? B * M * waves_per_query : 1);
  if (ns < 1) ns = 1;
  if (ns > chunks) ns = chunks;
  if (ns > 64) ns = 64;
  return static_cast<int>(ns);
}

template <int DQK, int DV>
struct SaLds {
  static constexpr int kRowStride = DQK + 8;  // bf16 elements per padded K row (+16 bytes)
  uint16_t krm[kKC * kRowStride];
  uint16_t vil[kKC * DV];  // [key/8][d][key%8]
  int32_t rows[kKC];       // gathered row index, -1 = invalid
};

template <int DQK, int DV>
__global__ __launch_bounds__(512) void sparse_attn_kernel(const uint16_t *__restrict__ q, const uint16_t *__restrict__ kv,
                                                         const float *__restrict__ sink, const int32_t *__restrict__ idx,
                                                         uint16_t *__restrict__ out, float *__restrict__ part_o,
                                                         float *__restrict__ part_ml, int64_t M, int64_t H, int64_t N,
                                                         int64_t K, int NS, int KR, float scale_log2) {
  using L = SaLds<DQK, DV>;
  constexpr int RS = L::kRowStride;
  constexpr int QJ = DQK / 32;  // k-steps of the QK MFMA
  constexpr int CT = DV / 16;   // dv column tiles
  __shared__ L lds;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nthreads = blockDim.x;
  const int split = blockIdx.x;
  const int64_t m = blockIdx.y, b = blockIdx.z;
  const int l16 = lane & 15, g = lane >> 4;
  const int head = wave * 16 + l16;  // head of this lane in the S^T / softmax layout
  const bool head_ok = head < H;
  const int64_t qm = b * M + m;

  // q B-fragments: Q[head][32j + 8g .. +7]
  uint4 qf[QJ];
#pragma unroll
  for (int j = 0; j < QJ; ++j)
    qf[j] = head_ok ? *reinterpret_cast<const uint4 *>(q + (qm * H + head) * DQK + 32 * j + 8 * g)
                    : make_uint4(0, 0, 0, 0);

  float run_max = -INFINITY, run_sum = 0.f;  // per head (lane l16), replicated over g
  f32x4_t o[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c) o[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int64_t k_begin = static_cast<int64_t>(split) * KR;
  const int64_t k_end = (k_begin + KR < K) ? k_begin + KR : K;
  const int32_t *irow = idx + qm * K;
  const uint16_t *kvb = kv + b * N * DQK;

  for (int64_t c0 = k_begin; c0 < k_end; c0 += kKC) {
    // ---- indices of this chunk
    if (tid < kKC) {
      const int64_t t = c0 + tid;
      int32_t r = t < k_end ? irow[t] : -1;
      if (r < 0 || r >= N) r = -1;
      lds.rows[tid] = r;
    }
    __syncthreads();
    // ---- gather: K row-major (padded) and V key-interleaved
    constexpr int UPR = DQK / 8;  // 16-byte units per row
    for (int u = tid; u < kKC * UPR; u += nthreads) {
      const int key = u / UPR, ch = u % UPR;
      const int32_t r = lds.rows[key];
      uint4 v = make_uint4(0, 0, 0, 0);
      if (r >= 0) v = *reinterpret_cast<const uint4 *>(kvb + static_cast<int64_t>(r) * DQK + ch * 8);
      *reinterpret_cast<uint4 *>(&lds.krm[key * RS + ch * 8]) = v;
      if (ch * 8 < DV) {
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
        uint16_t *dstv = &lds.vil[(key >> 3) * (DV * 8) + (ch * 8) * 8 + (key & 7)];
#pragma unroll
        for (int e = 0; e < 8; ++e) dstv[e * 8] = static_cast<uint16_t>(e & 1 ? (w4[e >> 1] >> 16) : (w4[e >> 1] & 0xFFFFu));
      }
    }
    __syncthreads();

    // ---- S^T = K Q^T for two 16-key tiles
    f32x4_t st[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      st[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const int key = 16 * t + l16;
#pragma unroll
      for (int j = 0; j < QJ; ++j) {
        const uint4 a = *reinterpret_cast<const uint4 *>(&lds.krm[key * RS + 32 * j + 8 * g]);
        st[t] = mfma16(a, qf[j], st[t]);
      }
    }
    // lane holds keys 16t + 4g + r for head l16
    float p[8];
    float cmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = lds.rows[16 * t + 4 * g + r] >= 0;
        const float sv = ok ? st[t][r] * scale_log2 : -INFINITY;
        p[4 * t + r] = sv;
        cmax = fmaxf(cmax, sv);
      }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
    const float new_max = fmaxf(run_max, cmax);
    const float alpha = (new_max == -INFINITY) ? 1.f : exp2f(run_max - new_max);
    float csum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = (p[i] == -INFINITY) ? 0.f : exp2f(p[i] - new_max);
      csum += p[i];
    }
    csum += __shfl_xor(csum, 16, 64);
    csum += __shfl_xor(csum, 32, 64);
    run_sum = run_sum * alpha + csum;
    run_max = new_max;
    // rescale O rows (heads 4g + r of this wave): alpha lives in lane l16 = 4g + r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ar = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
      for (int c = 0; c < CT; ++c) o[c][r] *= ar;
    }
    // ---- O += P V
    const uint4 pa = make_uint4(pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(p[4], p[5]),
                                pack_bf16x2(p[6], p[7]));
    const int grp0 = g >> 1, off = 4 * (g & 1);
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const int col = 16 * c + l16;
      const uint2 v0 = *reinterpret_cast<const uint2 *>(&lds.vil[grp0 * (DV * 8) + col * 8 + off]);
      const uint2 v1 = *reinterpret_cast<const uint2 *>(&lds.vil[(grp0 + 2) * (DV * 8) + col * 8 + off]);
      o[c] = mfma16(pa, make_uint4(v0.x, v0.y, v1.x, v1.y), o[c]);
    }
    __syncthreads();  // LDS is refilled by the next chunk
  }

  // ---- finalise: O rows are heads 4g + r; their (max, sum) live in lanes 4g + r
  if (NS == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hr = wave * 16 + 4 * g + r;
      const float mx = __shfl(run_max, 4 * g + r, 64);
      const float sm = __shfl(run_sum, 4 * g + r, 64);
      if (hr < H) {
        const float sk = sink[hr] * kLog2e;
        const float zmax = fmaxf(mx, sk);
        float scale_o = 0.f;
        if (zmax != -INFINITY) {
          const float e = (mx == -INFINITY) ? 0.f : exp2f(mx - zmax);
          const float den = sm * e + exp2f(sk - zmax);
          scale_o = den > 0.f ? e / den : 0.f;
        }
        uint16_t *orow = out + (qm * H + hr) * DV;
#pragma unroll
        for (int c = 0; c < CT; ++c) orow[16 * c + l16] = f32_to_bf16_rne(o[c][r] * scale_o);
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hr = wave * 16 + 4 * g + r;
      if (hr < H) {
        float *po = part_o + ((qm * NS + split) * H + hr) * DV;
#pragma unroll
        for (int c = 0; c < CT; ++c) po[16 * c + l16] = o[c][r];
      }
    }
    if (g == 0 && head_ok) {
      float *pml = part_ml + ((qm * NS + split) * H + head) * 2;
      pml[0] = run_max;
      pml[1] = run_sum;
    }
  }
}

// Merge NS partial ranges per (query, head) with the sink: one thread per output element.
__global__ __launch_bounds__(256) void sparse_attn_combine_kernel(const float *__restrict__ part_o,
                                                                 const float *__restrict__ part_ml,
                                                                 const float *__restrict__ sink,
                                                                 uint16_t *__restrict__ out, int64_t QH, int64_t H,
                                                                 int DV, int NS) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= QH * DV) return;
  const int64_t qh = e / DV;
  const int col = static_cast<int>(e % DV);
  const int64_t qi = qh / H, h = qh % H;
  const float sk = sink[h] * kLog2e;
  float zmax = sk;
  for (int s = 0; s < NS; ++s) zmax = fmaxf(zmax, part_ml[((qi * NS + s) * H + h) * 2]);
  float den = 0.f, acc = 0.f;
  if (zmax != -INFINITY) {
    den = exp2f(sk - zmax);
    for (int s = 0; s < NS; ++s) {
      const int64_t base = (qi * NS + s) * H + h;
      const float mx = part_ml[base * 2];
      if (mx == -INFINITY) continue;
      const float w = exp2f(mx - zmax);
      den += part_ml[base * 2 + 1] * w;
      acc += part_o[base * DV + col] * w;
    }
  }
  out[e] = f32_to_bf16_rne(den > 0.f ? acc / den : 0.f);
}

template <int DQK, int DV>
int launch_sa(const uint16_t *q, const uint16_t *kv, const float *sink, const int32_t *idx, uint16_t *out,
              int64_t B, int64_t M, int64_t H, int64_t N, int64_t K, float scale, void *ws, hipStream_t stream) {
  const int NS = choose_splits(B, M, H, K);
  const int64_t chunks = (K + kKC - 1) / kKC;
  const int KR = static_cast<int>(((chunks + NS - 1) / NS) * kKC);
  const int nsplit = static_cast<int>((K + KR - 1) / KR);  // ranges actually used
  float *part_o = nullptr, *part_ml = nullptr;
  if (nsplit > 1) {
    part_o = static_cast<float *>(ws);
    part_ml = part_o + B * M * nsplit * H * DV;
  }
  const int waves = static_cast<int>((H + 15) / 16);
  dim3 grid(static_cast<unsigned>(nsplit), static_cast<unsigned>(M), static_cast<unsigned>(B));
  hipLaunchKernelGGL((sparse_attn_kernel<DQK, DV>), grid, dim3(64 * waves), 0, stream, q, kv, sink, idx, out, part_o,
                     part_ml, M, H, N, K, nsplit, KR, scale * kLog2e);
  KS_CHECK_LAUNCH("sparse_attn_kernel");
  if (nsplit > 1) {
    const int64_t total = B * M * H * DV;
    hipLaunchKernelGGL(sparse_attn_combine_kernel, dim3(static_cast<unsigned>(ceil_div(total, 256))), dim3(256), 0,
                       stream, part_o, part_ml, sink, out, B * M * H, H, DV, nsplit);
    KS_CHECK_LAUNCH("sparse_attn_combine_kernel");
  }
  return KS_OK;
}

size_t sa_workspace(int64_t B, int64_t M, int64_t H, int64_t K, int64_t DV) {
  const int NS = choose_splits(B, M, H, K);
  const int64_t chunks = (K + kKC - 1) / kKC;
  const int64_t KR = ((chunks + NS - 1) / NS) * kKC;
  const int64_t nsplit = (K + KR - 1) / KR;
  if (nsplit <= 1) return 0;
  return static_cast<size_t>(B * M * nsplit * H * (DV + 2)) * sizeof(float);
}

}  // namespace
}  // namespace ks

extern "C" size_t ks_sparse_attn_workspace_size(int64_t B, int64_t M, int64_t H, int64_t Dqk, int64_t Dv, int64_t K) {
  (void)Dqk;
  if (B <= 0 || M <= 0 || H <= 0 || K <= 0 || Dv <= 0) return 0;
  return ks::sa_workspace(B, M, H, K, Dv);
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
  if (B * M == 0) return KS_OK;
  KS_CHECK_ARG(q && kv && sink && idx && out, "ks_sparse_attn: null pointer");
  KS_CHECK_ARG(ks::aligned(q, 16) && ks::aligned(kv, 16), "ks_sparse_attn: q and kv must be 16-byte aligned");
  const size_t need = ks::sa_workspace(B, M, H, K, Dv);
  KS_CHECK_ARG(need == 0 || (workspace != nullptr && workspace_bytes >= need),
               "ks_sparse_attn: workspace of %zu bytes required, %zu given", need, workspace_bytes);
  KS_CHECK_ARG(need == 0 || ks::aligned(workspace, 16), "ks_sparse_attn: workspace must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d128) return ks::launch_sa<128, 128>(q, kv, sink, idx, out, B, M, H, N, K, scale, workspace, st);
  return ks::launch_sa<576, 512>(q, kv, sink, idx, out, B, M, H, N, K, scale, workspace, st);
}
