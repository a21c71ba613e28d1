// Flash-style relative-position multi-head self-attention on gfx950 MFMA.
//
// For head h, query q and key k of one sequence (length T):
//   s[q,k] = scale * ( (q+u)_q . K_k  +  (q+v)_q . relK[j] ),  j = tc-1-q+k
//   o[q]   = sum_k softmax_k(s[q,:]) V_k          (keys k >= T masked)
// which is the reference's content GEMM + windowed bd GEMM + fused
// rel-shift/softmax + AV GEMM (src/encoder.rs:2238-2347,
// src/encoder/shader_sources.rs:472-539; CPU: src/cpu/layer.rs:251-294,
// src/cpu/ops.rs:133-189) without any T x T buffer: the softmax is computed
// online over 64-key tiles. q+u and q+v arrive pre-multiplied by
// scale*log2(e) (qkv GEMM epilogue), so scores are already in the log2 domain.
//
// Work split: one workgroup = 128 queries of one (sequence, head); 8 waves.
// Wave w owns query group w&3 (32 queries) and key half w>>2 (32 keys) of every
// 64-key tile, keeping its own running max / sum / output; the two halves of a
// query group are merged at the end. Scores are computed transposed
// (S^T = K . Qu^T), so a lane's accumulator column is one query: the softmax
// max/sum need one cross-lane exchange (lane ^ 32), and the exp'd scores are
// already laid out as the B operand of the P.V MFMA (keys permuted
// consistently with the V^T fragment). The position term is a band product
// relK[jband] . Qv^T over the 64 relative positions a wave's 32 queries x 32
// keys touch (2x the in-band work), written to a per-wave LDS scratch and read
// back along the diagonal j = k + 31 - q_local — that read is the rel-shift.
// The relK band lives in LDS as a ring of six 32-row blocks, so each key tile
// fetches only its 64 new band rows; the next tile's K, V^T and new band rows
// are fetched into registers while the current tile computes.
//
// Inputs are f16: K, V and relK exactly as the reference rounds them
// (src/cpu/ops.rs:258-259, src/cpu/layer.rs:234-247); q+u and q+v rounded to
// f16 for the MFMA operand. Accumulation and softmax are f32.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "kernels.h"

namespace bark {
namespace {

constexpr int BQ = 128;
constexpr int BKV = 64;
constexpr int KLD = HDIM + 8;   // halves per LDS row of K and relK
constexpr int VLD = BKV + 8;    // halves per LDS row of V^T
constexpr int BAND = BQ + BKV;  // relK rows staged per key tile (191 used)
constexpr int PLD = 68;         // floats per row of a wave's band scratch (64 used)
constexpr int NT = 512;         // threads per workgroup

constexpr int K_CH = BKV * HDIM / 8 / NT;   // 16-byte chunks per thread
constexpr int V_CH = HDIM * BKV / 8 / NT;
constexpr int R_CH = BAND * HDIM / 8 / NT;

struct Smem {
  half K[BKV * KLD];
  half V[HDIM * VLD];
  half R[BAND * KLD];
  float P[8][32 * PLD];
};

__global__ void __launch_bounds__(NT) rel_attn_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  Smem& sm = *reinterpret_cast<Smem*>(smem_raw);

  // Workgroups are dispatched round-robin over the 8 XCDs, so block b runs on
  // XCD b % 8: giving head b % 8 to it keeps every query tile of one head on one
  // XCD, whose L2 then holds that head's K, V^T and relK (2.2 MB at T = 2207).
  const int h = blockIdx.x % HEADS;
  const int slot = blockIdx.x / HEADS;
  const int4 tile = a.tiles[slot];
  const int start = tile.x, T = tile.y, q0 = tile.z;
  const int k_begin = (tile.w & 0xffff) * BKV, k_end = min(T, (tile.w >> 16) * BKV);
  const bool complete = k_begin == 0 && k_end == T;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int qg = wid & 3, kh = wid >> 2;
  const int l32 = lane & 31, lhi = lane >> 5;
  const int q_lane = q0 + 32 * qg + l32;
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
  float* ps = sm.P[wid];
  const uint4 zero4 = {0u, 0u, 0u, 0u};

  // Per-thread chunk coordinates (loop invariant). K and the relK rows: 16
  // chunks of 8 halves per row; V^T: 8 chunks of 8 keys per d-row.
  int k_row[K_CH], v_d[V_CH], v_kc[V_CH], r_row[2];
  const int col16 = (tid & 15) * 8;
#pragma unroll
  for (int i = 0; i < K_CH; ++i) k_row[i] = (tid + NT * i) >> 4;
#pragma unroll
  for (int i = 0; i < V_CH; ++i) {
    v_d[i] = (tid + NT * i) >> 3;
    v_kc[i] = ((tid + NT * i) & 7) * 8;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) r_row[i] = (tid + NT * i) >> 4;

  // relK band as a ring of 6 blocks of 32 rows: band row r of this
  // workgroup's key tile t (t = 0 at k_begin) lives in block ((r >> 5) + 2t) % 6.
  // Each tile only fetches its last 64 rows (the first 128 are the previous
  // tile's last 128). The band of the tile at key k0 starts at row jg00 + k0.
  const int jg00 = a.tc - 1 - (q0 + BQ - 1);
  auto r_ok = [&](int j) { return j >= 0 && j < prows; };
  for (int i = 0; i < R_CH; ++i) {  // first tile: all 192 rows
    const int ch = tid + NT * i, row = ch >> 4;
    const int j = jg00 + k_begin + row;
    const uint4 v = r_ok(j) ? *reinterpret_cast<const uint4*>(rbase + (size_t)j * HDIM + col16) : zero4;
    *reinterpret_cast<uint4*>(&sm.R[row * KLD + col16]) = v;
  }

  uint4 kr[K_CH], vr[V_CH], rr[2];
  auto fetch = [&](int k0, int t) {
    const bool interior = k0 + BKV <= T;
    if (interior) {
#pragma unroll
      for (int i = 0; i < K_CH; ++i)
        kr[i] = *reinterpret_cast<const uint4*>(kbase + (size_t)(k0 + k_row[i]) * HDIM + col16);
#pragma unroll
      for (int i = 0; i < V_CH; ++i)
        vr[i] = *reinterpret_cast<const uint4*>(vbase + (size_t)v_d[i] * a.mp + k0 + v_kc[i]);
    } else {
#pragma unroll
      for (int i = 0; i < K_CH; ++i)
        kr[i] = (k0 + k_row[i] < T)
                    ? *reinterpret_cast<const uint4*>(kbase + (size_t)(k0 + k_row[i]) * HDIM + col16)
                    : zero4;
#pragma unroll
      for (int i = 0; i < V_CH; ++i) {
        uint4 v = zero4;
        const int kc = v_kc[i];
        if (k0 + kc < T) {
          v = *reinterpret_cast<const uint4*>(vbase + (size_t)v_d[i] * a.mp + k0 + kc);
          if (k0 + kc + 8 > T) {  // zero the keys past the sequence end
            half8 hv = *reinterpret_cast<half8*>(&v);
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (k0 + kc + e >= T) hv[e] = (half)0.0f;
            v = *reinterpret_cast<uint4*>(&hv);
          }
        }
        vr[i] = v;
      }
    }
    const int jn = jg00 + k0 + 128;  // first new band row of the tile at k0
    if (jn >= 0 && jn + 64 <= prows) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        rr[i] = *reinterpret_cast<const uint4*>(rbase + (size_t)(jn + r_row[i]) * HDIM + col16);
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int j = jn + r_row[i];
        rr[i] = r_ok(j) ? *reinterpret_cast<const uint4*>(rbase + (size_t)j * HDIM + col16) : zero4;
      }
    }
  };
  auto stage = [&](int t) {
#pragma unroll
    for (int i = 0; i < K_CH; ++i) *reinterpret_cast<uint4*>(&sm.K[k_row[i] * KLD + col16]) = kr[i];
#pragma unroll
    for (int i = 0; i < V_CH; ++i) *reinterpret_cast<uint4*>(&sm.V[v_d[i] * VLD + v_kc[i]]) = vr[i];
    if (t > 0) {  // new band rows 128..191 of tile t -> ring blocks (4,5) + 2t
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = 128 + r_row[i];
        const int prow = (((r >> 5) + 2 * t) % 6) * 32 + (r & 31);
        *reinterpret_cast<uint4*>(&sm.R[prow * KLD + col16]) = rr[i];
      }
    }
  };

  const int rb0 = 96 - 32 * qg + 32 * kh;  // first band row of this wave
  fetch(k_begin, 0);
  int t = 0;
  for (int k0 = k_begin; k0 < k_end; k0 += BKV, ++t) {
    stage(t);
    __syncthreads();
    if (k0 + BKV < k_end) fetch(k0 + BKV, t + 1);

    // ---- content scores S^T (this wave's 32 keys x 32 queries) and the
    // position band relK[j] . Qv^T over the wave's 64 band rows: three
    // independent MFMA chains, interleaved so they overlap in the pipeline
    floatx16 s, bd0, bd1;
#pragma unroll
    for (int v = 0; v < 16; ++v) s[v] = bd0[v] = bd1[v] = 0.0f;
    const int pb0 = ((rb0 >> 5) + 2 * t) % 6, pb1 = ((rb0 >> 5) + 1 + 2 * t) % 6;  // ring blocks
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const half8 kf = ld_half8(&sm.K[(32 * kh + l32) * KLD + 16 * st + 8 * lhi]);
      const half8 r0 = ld_half8(&sm.R[(pb0 * 32 + l32) * KLD + 16 * st + 8 * lhi]);
      const half8 r1 = ld_half8(&sm.R[(pb1 * 32 + l32) * KLD + 16 * st + 8 * lhi]);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, quf[st], s, 0, 0, 0);
      bd0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(r0, qvf[st], bd0, 0, 0, 0);
      bd1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(r1, qvf[st], bd1, 0, 0, 0);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const floatx4 w0 = {bd0[4 * g], bd0[4 * g + 1], bd0[4 * g + 2], bd0[4 * g + 3]};
      const floatx4 w1 = {bd1[4 * g], bd1[4 * g + 1], bd1[4 * g + 2], bd1[4 * g + 3]};
      *reinterpret_cast<floatx4*>(&ps[l32 * PLD + 8 * g + 4 * lhi]) = w0;
      *reinterpret_cast<floatx4*>(&ps[l32 * PLD + 32 + 8 * g + 4 * lhi]) = w1;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- rel-shift (diagonal read), mask, online softmax (log2 domain)
    const bool tail = k0 + BKV > T;
    float mt = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int kk = 8 * (v >> 2) + 4 * lhi + (v & 3);  // key within the wave's half
      float x = s[v] + ps[l32 * PLD + kk + 31 - l32];
      if (tail && k0 + 32 * kh + kk >= T) x = -INFINITY;
      s[v] = x;
      mt = fmaxf(mt, x);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    // Lazy rescaling: exp2 is taken against a reference max m_run that is only
    // raised when a new score exceeds it by more than 8 (log2 units), so
    // p <= 256 and the output/sum rescale runs rarely. Softmax is invariant to
    // the reference, so this is exact up to rounding.
    if (__any(mt > m_run + 8.0f)) {
      const float m_new = fmaxf(m_run, mt);
      const float corr = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= corr;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] *= corr;
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;  // a half with no valid key yet
    float ls = 0.0f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float pv = __builtin_amdgcn_exp2f(s[v] - m_use);
      s[v] = pv;
      ls += pv;
    }
    ls += __shfl_xor(ls, 32, 64);
    l_run += ls;

    // ---- O^T (128 d x 32 q) += V^T . P^T over this wave's 32 keys
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      half8 pf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pf[e] = (half)s[8 * st + e];
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const half* vp = &sm.V[(32 * db + l32) * VLD + 32 * kh + 16 * st + 4 * lhi];
        const half4 lo = *reinterpret_cast<const half4*>(vp);
        const half4 hi = *reinterpret_cast<const half4*>(vp + 8);
        const half8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, o[db], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // ---- merge the two key halves of each query group (through LDS), write out
  float* xo = reinterpret_cast<float*>(sm.K);  // reuses the K/V/relK staging area
  float* xm = xo + 4 * 64 * 64;
  if (kh == 1) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int v = 0; v < 16; ++v) xo[(qg * 64 + db * 16 + v) * 64 + lane] = o[db][v];
    xm[(qg * 2) * 64 + lane] = m_run;
    xm[(qg * 2 + 1) * 64 + lane] = l_run;
  }
  __syncthreads();
  if (kh == 0 && !complete) {  // partial over this key range: o unnormalised, with its max and sum
    const float m1 = xm[(qg * 2) * 64 + lane], l1 = xm[(qg * 2 + 1) * 64 + lane];
    const float m = fmaxf(m_run, m1);
    const float c0 = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
    const float c1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - m);
    const int ql = 32 * qg + l32;
    const size_t sh = (size_t)slot * HEADS + h;
    float* po = a.part_o + (sh * BQ + ql) * HDIM;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        floatx4 w4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = 4 * g + i;
          w4[i] = o[db][v] * c0 + xo[(qg * 64 + db * 16 + v) * 64 + lane] * c1;
        }
        *reinterpret_cast<floatx4*>(po + 32 * db + 8 * g + 4 * lhi) = w4;
      }
    if (lhi == 0) {
      float* pm = a.part_ml + (sh * BQ + ql) * 2;
      pm[0] = m;
      pm[1] = l_run * c0 + l1 * c1;
    }
  }
  if (kh == 0 && complete && q_lane < T) {
    const float m1 = xm[(qg * 2) * 64 + lane], l1 = xm[(qg * 2 + 1) * 64 + lane];
    const float m = fmaxf(m_run, m1);
    const float c0 = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
    const float c1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - m);
    const float inv = 1.0f / (l_run * c0 + l1 * c1);
    half* orow = a.out + (size_t)(start + q_lane) * HIDDEN + h * HDIM;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        half4 w4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = 4 * g + i;
          w4[i] = (half)((o[db][v] * c0 + xo[(qg * 64 + db * 16 + v) * 64 + lane] * c1) * inv);
        }
        *reinterpret_cast<half4*>(orow + 32 * db + 8 * g + 4 * lhi) = w4;
      }
  }
}

// Combines the key-range partials of one (query tile, head): with weights
// w_s = 2^(m_s - max_s m_s), out = sum_s w_s o_s / sum_s w_s l_s, slots in
// order. Thread t handles query t/2, dims 64*(t&1) .. +63.
__global__ void __launch_bounds__(256) attn_merge_kernel(const float* part_o, const float* part_ml,
                                                         const int4* merges, half* out) {
  const int h = blockIdx.x % HEADS;
  const int4 mg = merges[blockIdx.x / HEADS];
  const int q = threadIdx.x >> 1, d0 = (threadIdx.x & 1) * 64;
  if (q >= mg.w) return;
  float m = -INFINITY;
  for (int s = 0; s < mg.y; ++s)
    m = fmaxf(m, part_ml[(((size_t)(mg.x + s) * HEADS + h) * BQ + q) * 2]);
  float o[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) o[i] = 0.0f;
  float l = 0.0f;
  for (int s = 0; s < mg.y; ++s) {
    const size_t sh = ((size_t)(mg.x + s) * HEADS + h) * BQ + q;
    const float w = __builtin_amdgcn_exp2f(part_ml[sh * 2] - m);
    l += w * part_ml[sh * 2 + 1];
    const floatx4* src = reinterpret_cast<const floatx4*>(part_o + sh * HDIM + d0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const floatx4 v = src[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[4 * i + e] += w * v[e];
    }
  }
  const float inv = 1.0f / l;
  half* dst = out + (size_t)(mg.z + q) * HIDDEN + h * HDIM + d0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const half4 w4 = {(half)(o[4 * i] * inv), (half)(o[4 * i + 1] * inv), (half)(o[4 * i + 2] * inv),
                      (half)(o[4 * i + 3] * inv)};
    *reinterpret_cast<half4*>(dst + 4 * i) = w4;
  }
}

}  // namespace

int attention_splits(int t) {
  static const int forced = [] {
    const char* e = getenv("BARK_HIP_ATTN_SPLITS");
    return e ? atoi(e) : 0;
  }();
  const int qt = (t + BQ - 1) / BQ, ntk = (t + BKV - 1) / BKV;
  if (forced > 0) return std::min(forced, ntk);
  // Workgroups of one sequence = query tiles x heads x splits on 256 CUs (one
  // workgroup each): pick the split count whose launch leaves the fewest
  // slots idle, counting every round, with a small cost per extra split.
  int best = 1;
  double best_score = -1.0;
  for (int s = 1; s <= std::min(8, ntk); ++s) {
    const long w = (long)qt * HEADS * s;
    const long rounds = (w + 255) / 256;
    const double score = (double)w / (256.0 * rounds) - 0.06 * (s - 1);
    if (score > best_score + 1e-9) {
      best_score = score;
      best = s;
    }
  }
  return best;
}

void rel_attention(const AttnArgs& a, hipStream_t stream) {
  BARK_REQUIRE(a.ntiles > 0 && a.tiles, "rel_attention: no query tiles");
  BARK_REQUIRE(a.mp % 64 == 0 && a.pp >= 2 * a.tc - 1, "rel_attention: bad buffer shape");
  static_assert(sizeof(Smem) <= 160 * 1024, "LDS budget");
  static_assert(4 * 64 * 64 * 4 + 8 * 64 * 4 <= BKV * KLD * 2 + HDIM * VLD * 2 + BAND * KLD * 2,
                "merge area must fit in the staging area");
  static bool attr = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(rel_attn_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, sizeof(Smem)) == hipSuccess;
  }();
  BARK_REQUIRE(attr, "rel_attention: cannot reserve LDS");
  BARK_REQUIRE(a.nmerges == 0 || (a.merges && a.part_o && a.part_ml), "rel_attention: missing partial buffers");
  hipLaunchKernelGGL(rel_attn_kernel, dim3(a.ntiles * HEADS), dim3(NT), sizeof(Smem), stream, a);
  BARK_HIP_CHECK(hipGetLastError());
  if (a.nmerges > 0) {
    hipLaunchKernelGGL(attn_merge_kernel, dim3(a.nmerges * HEADS), dim3(256), 0, stream, a.part_o, a.part_ml,
                       a.merges, a.out);
    BARK_HIP_CHECK(hipGetLastError());
  }
}

// scale * log2(e) applied to q+u and q+v by the qkv epilogue
float attention_q_scale() { return (1.0f / sqrtf((float)HDIM)) * 1.4426950408889634f; }

}  // namespace bark
