// Flash-style relative-position multi-head self-attention on gfx950 MFMA.
//
// For head h, query q and key k of one sequence (length T):
//   s[q,k] = scale * ( (q+u)_q . K_k  +  (q+v)_q . relK[j] ),  j = tc-1-q+k
//   o[q]   = sum_k softmax_k(s[q,:]) V_k          (keys k >= T masked)
// which is the reference's content GEMM + windowed bd GEMM + fused
// rel-shift/softmax + AV GEMM (src/encoder.rs:2238-2347,
// src/encoder/shader_sources.rs:472-539; CPU: src/cpu/layer.rs:251-294,
// src/cpu/ops.rs:133-189) without any T x T buffer: the softmax is computed
// online over 64-key tiles.
//
// Work split: one workgroup = 128 queries of one (sequence, head); 4 waves,
// each owning 32 queries. Scores are computed transposed (S^T = K . Qu^T), so
// a lane's accumulator column is one query: the softmax max/sum need only one
// cross-lane exchange (lane ^ 32), and the exp'd scores are already laid out
// as the B operand of the P.V MFMA (keys permuted consistently with the V^T
// fragment). The position term is computed as a band product
// relK[jband] . Qv^T (96 positions x 32 queries per wave, 1.5x the in-band
// work), written to a per-wave LDS scratch and read back along the diagonal
// j = k + 31 - q_local — that read is the rel-shift.
//
// Inputs are f16: K, V and relK exactly as the reference rounds them
// (src/cpu/ops.rs:258-259, src/cpu/layer.rs:234-247); q+u and q+v rounded to
// f16 for the MFMA operand. Accumulation and softmax are f32.
#include <cmath>

#include "kernels.h"

namespace bark {
namespace {

constexpr int BQ = 128;
constexpr int BKV = 64;
constexpr int KLD = HDIM + 8;  // halves per LDS row of K and relK
constexpr int VLD = BKV + 8;   // halves per LDS row of V^T
constexpr int BAND = BQ + BKV; // relK rows staged per key tile (191 used)
constexpr int PLD = 100;       // floats per row of the band scratch (96 used)

__global__ void __launch_bounds__(256) rel_attn_kernel(AttnArgs a, float scale_log2) {
  __shared__ __attribute__((aligned(16))) half K_s[BKV * KLD];
  __shared__ __attribute__((aligned(16))) half V_s[HDIM * VLD];
  __shared__ __attribute__((aligned(16))) half R_s[BAND * KLD];
  __shared__ __attribute__((aligned(16))) float P_s[4][32 * PLD];

  const int4 tile = a.tiles[blockIdx.x];
  const int start = tile.x, T = tile.y, q0 = tile.z;
  const int h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, lhi = lane >> 5;
  const int q_lane = q0 + 32 * wid + l32;
  const int prows = 2 * a.tc - 1;

  // B-operand fragments of Qu^T / Qv^T: lane holds q_lane, dims 16s+8*lhi..+7.
  half8 quf[8], qvf[8];
  if (q_lane < T) {
    const size_t off = ((size_t)h * a.mp + start + q_lane) * HDIM + 8 * lhi;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      quf[s] = ld_half8(a.qu + off + 16 * s);
      qvf[s] = ld_half8(a.qv + off + 16 * s);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) quf[s][e] = qvf[s][e] = (half)0.0f;
  }

  floatx16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  const half* kbase = a.kh + ((size_t)h * a.mp + start) * HDIM;
  const half* vbase = a.vt + (size_t)h * HDIM * a.mp + start;
  const half* rbase = a.rk + (size_t)h * a.pp * HDIM;
  float* ps = P_s[wid];
  const uint4 zero4 = {0u, 0u, 0u, 0u};

  for (int k0 = 0; k0 < T; k0 += BKV) {
    // ---- stage K (64 x 128), V^T (128 x 64) and the relK band (192 x 128)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + 256 * i, row = ch >> 4, col = (ch & 15) * 8;
      uint4 v = zero4;
      if (k0 + row < T) v = *reinterpret_cast<const uint4*>(kbase + (size_t)(k0 + row) * HDIM + col);
      *reinterpret_cast<uint4*>(&K_s[row * KLD + col]) = v;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + 256 * i, d = ch >> 3, kc = (ch & 7) * 8;
      uint4 v = zero4;
      if (k0 + kc < T) {
        v = *reinterpret_cast<const uint4*>(vbase + (size_t)d * a.mp + k0 + kc);
        if (k0 + kc + 8 > T) {  // zero the keys past the sequence end
          half8 hv = *reinterpret_cast<half8*>(&v);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (k0 + kc + e >= T) hv[e] = (half)0.0f;
          v = *reinterpret_cast<uint4*>(&hv);
        }
      }
      *reinterpret_cast<uint4*>(&V_s[d * VLD + kc]) = v;
    }
    const int jg0 = a.tc - 1 - (q0 + BQ - 1) + k0;
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      const int ch = tid + 256 * i, row = ch >> 4, col = (ch & 15) * 8;
      const int j = jg0 + row;
      uint4 v = zero4;
      if (j >= 0 && j < prows) v = *reinterpret_cast<const uint4*>(rbase + (size_t)j * HDIM + col);
      *reinterpret_cast<uint4*>(&R_s[row * KLD + col]) = v;
    }
    __syncthreads();

    // ---- content scores S^T (64 keys x 32 queries)
    floatx16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) s[kb][v] = 0.0f;
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const half8 kf = ld_half8(&K_s[(kb * 32 + l32) * KLD + 16 * st + 8 * lhi]);
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, quf[st], s[kb], 0, 0, 0);
      }
    }
    // ---- position band relK[j] . Qv^T over this wave's 96 band rows
    const int rb0 = 96 - 32 * wid;
#pragma unroll
    for (int bb = 0; bb < 3; ++bb) {
      floatx16 bd;
#pragma unroll
      for (int v = 0; v < 16; ++v) bd[v] = 0.0f;
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const half8 rf = ld_half8(&R_s[(rb0 + bb * 32 + l32) * KLD + 16 * st + 8 * lhi]);
        bd = __builtin_amdgcn_mfma_f32_32x32x16_f16(rf, qvf[st], bd, 0, 0, 0);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        floatx4 w4 = {bd[4 * g], bd[4 * g + 1], bd[4 * g + 2], bd[4 * g + 3]};
        *reinterpret_cast<floatx4*>(&ps[l32 * PLD + 32 * bb + 8 * g + 4 * lhi]) = w4;
      }
    }
    __syncthreads();

    // ---- rel-shift + scale + mask, online softmax
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int kk = 32 * kb + 8 * (v >> 2) + 4 * lhi + (v & 3);
        float x = (s[kb][v] + ps[l32 * PLD + kk + 31 - l32]) * scale_log2;
        if (k0 + kk >= T) x = -INFINITY;
        s[kb][v] = x;
        mt = fmaxf(mt, x);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);
    const float corr = exp2f(m_run - m_new);
    float ls = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float pv = exp2f(s[kb][v] - m_new);
        s[kb][v] = pv;
        ls += pv;
      }
    ls += __shfl_xor(ls, 32, 64);
    l_run = l_run * corr + ls;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[db][v] *= corr;

    // ---- O^T (128 d x 32 q) += V^T . P^T over 4 steps of 16 keys
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int kb = st >> 1, vb = 8 * (st & 1);
      half8 pf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[e] = (half)s[kb][vb + e];
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const half* vp = &V_s[(32 * db + l32) * VLD + 16 * st + 4 * lhi];
        const half4 lo = *reinterpret_cast<const half4*>(vp);
        const half4 hi = *reinterpret_cast<const half4*>(vp + 8);
        const half8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, o[db], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  if (q_lane < T) {
    const float inv = 1.0f / l_run;
    half* orow = a.out + (size_t)(start + q_lane) * HIDDEN + h * HDIM;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const half4 w4 = {(half)(o[db][4 * g] * inv), (half)(o[db][4 * g + 1] * inv),
                          (half)(o[db][4 * g + 2] * inv), (half)(o[db][4 * g + 3] * inv)};
        *reinterpret_cast<half4*>(orow + 32 * db + 8 * g + 4 * lhi) = w4;
      }
  }
}

}  // namespace

void rel_attention(const AttnArgs& a, hipStream_t stream) {
  BARK_REQUIRE(a.ntiles > 0 && a.tiles, "rel_attention: no query tiles");
  BARK_REQUIRE(a.mp % 64 == 0 && a.pp >= 2 * a.tc - 1, "rel_attention: bad buffer shape");
  const float scale_log2 = (1.0f / sqrtf((float)HDIM)) * 1.4426950408889634f;
  hipLaunchKernelGGL(rel_attn_kernel, dim3(a.ntiles, HEADS), dim3(256), 0, stream, a,
                     scale_log2);
  BARK_HIP_CHECK(hipGetLastError());
}

}  // namespace bark
