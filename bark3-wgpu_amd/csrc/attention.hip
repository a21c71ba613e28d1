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
// Work split: one workgroup per (lane, head) runs its lane's segments, each
// 128 queries of one sequence over a range of 64-key tiles (the whole
// sequence, or a piece whose partial is merged later); the host spreads a
// sequence's query tile x key tile units evenly over its lanes, so one launch
// fills the CUs in one round. 4 waves: wave w owns queries 32w .. 32w+31 against
// all 64 keys of every key tile, with its own running max / sum / output. Scores are
// computed transposed (S^T = K . Qu^T, two 32-key blocks), so a lane's
// accumulator column is one query: the softmax max/sum need one cross-lane
// exchange (lane ^ 32), and the exp'd scores are already laid out as the B
// operand of the P.V MFMA (keys permuted consistently with the V^T fragment).
// The position term is a band product relK[jband] . Qv^T over the 96 relative
// positions a wave's 32 queries x 64 keys touch (1.5x the in-band work),
// written to a per-wave LDS scratch and read back along the diagonal
// j = k + 31 - q_local — that read is the rel-shift. The relK band lives in
// LDS as a ring of six 32-row blocks, so each key tile fetches only its 64 new
// band rows; the next tile's K, V^T and new band rows are loaded into
// registers while the current tile computes (four waves per workgroup leave
// each wave 512 registers, so nothing spills).
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
constexpr int PLD = 100;        // floats per row of a wave's band scratch (96 used)
constexpr int NT = 256;         // threads per workgroup

constexpr int K_CH = BKV * HDIM / 8 / NT;   // 16-byte chunks per thread
constexpr int V_CH = HDIM * BKV / 8 / NT;
constexpr int R_NEW = 64 * HDIM / 8 / NT;   // new band rows per tile
constexpr int R_CH = BAND * HDIM / 8 / NT;

// Register-class pins (empty asm): keep a value in the accumulation registers
// (AGPRs: the output accumulators, which MFMA updates in place) or in the
// vector registers (values the VALU works on). Without them the allocator
// copies the 64 output accumulators between the two files every key tile. (A
// pin makes the value ready at that point, so it never goes on a load.)
template <typename T>
__device__ inline void pin_acc(T& x) {
  asm volatile("" : "+a"(x));
}
template <typename T>
__device__ inline void pin_vgpr(T& x) {
  asm volatile("" : "+v"(x));
}

// max / sum of x over lanes l and l ^ 32 (one cross-half swap, no LDS trip)
__device__ inline float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 16 bytes at base + byte offset off (a uniform base and a 32-bit lane offset)
__device__ inline uint4 ld_u4(const half* base, uint32_t off) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + off);
}

struct Smem {
  half K[BKV * KLD];
  half V[HDIM * VLD];
  half R[BAND * KLD];
  float P[4][32 * PLD];
};

__global__ void __launch_bounds__(NT) rel_attn_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  Smem& sm = *reinterpret_cast<Smem*>(smem_raw);

  // Workgroups are dispatched round-robin over the 8 XCDs, so block b runs on
  // XCD b % 8: giving head b % 8 to it keeps every query tile of one head on one
  // XCD, whose L2 then holds that head's K, V^T and relK (2.2 MB at T = 2207).
  const int h = blockIdx.x % HEADS;
  const int wl = blockIdx.x / HEADS;  // workgroup lane
  const int tid = threadIdx.x, lane = tid & 63;
  const int qg = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index (uniform)
  const int l32 = lane & 31, lhi = lane >> 5;
  const int seg_end = a.lanes[wl + 1];
  for (int slot = a.lanes[wl]; slot < seg_end; ++slot) {
    const int4 tile = a.tiles[slot];
    const int start = tile.x, T = tile.y, q0 = tile.z;
    const int k_begin = (tile.w & 0xffff) * BKV, k_end = min(T, (tile.w >> 16) * BKV);
    const bool complete = k_begin == 0 && k_end == T;
    const int q_lane = q0 + 32 * qg + l32;
    const int prows = 2 * a.tc - 1;

    // B-operand fragments of Qu^T / Qv^T: lane holds q_lane, dims 16s+8*lhi..+7
    // (zero past the sequence end). Loads and arrays stay branch-free
    // throughout so the compiler keeps the arrays in registers.
    half8 quf[8], qvf[8];
    {
      const bool qv_ok = q_lane < T;
      const size_t off = ((size_t)h * a.mp + start + min(q_lane, T - 1)) * HDIM + 8 * lhi;
      const half8 z8 = {};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const half8 u = ld_half8(a.qu + off + 16 * s), v = ld_half8(a.qv + off + 16 * s);
        quf[s] = qv_ok ? u : z8;
        qvf[s] = qv_ok ? v : z8;
      }
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
    float* ps = sm.P[qg];

    // Per-thread chunk coordinates (loop invariant). K and relK rows: 16 chunks
    // of 8 halves per row; V^T: 8 chunks of 8 keys per d-row.
    const int col16 = (tid & 15) * 8;
    const int row16 = tid >> 4;        // + 16 i
    const int v_d = tid >> 3;          // + 32 i
    const int v_kc = (tid & 7) * 8;

    // relK band as a ring of 6 blocks of 32 rows: band row r of this
    // workgroup's key tile t (t = 0 at k_begin) lives in block ((r >> 5) + 2t) % 6.
    // Each tile only fetches its last 64 rows (the first 128 are the previous
    // tile's last 128). The band of the tile at key k0 starts at row jg00 + k0.
    const int jg00 = a.tc - 1 - (q0 + BQ - 1);
#pragma unroll 4
    for (int i = 0; i < R_CH; ++i) {  // first tile: all 192 rows (row index clamped into the block)
      const int row = row16 + 16 * i;
      *reinterpret_cast<uint4*>(&sm.R[row * KLD + col16]) =
          *reinterpret_cast<const uint4*>(rbase + (size_t)min(max(jg00 + k_begin + row, 0), prows - 1) * HDIM + col16);
    }

    // The next key tile into registers. K rows and V^T columns past T stay inside
    // the sequence's 64-row-aligned slot of the packed buffers; they are zeroed
    // when staged (keys past T are also masked out of the softmax). The masks
    // are applied at staging, not here, so the loads stay in flight across the
    // current tile's work.
    uint4 kr[K_CH], vr[V_CH], rr[R_NEW];
    // Load n (0 .. 11) of the key tile at k0: K rows, V^T columns, new band rows.
    // Uniform tile bases (readfirstlane keeps the compiler from turning the
    // addresses into per-load 64-bit pointer recurrences) plus 32-bit lane byte
    // offsets; a head's block is < 2^31 elements (checked on the host).
    auto fetch_one = [&](int k0_, int n) {
      const int k0 = __builtin_amdgcn_readfirstlane(k0_);
      if (n < K_CH) {
        kr[n] = ld_u4(kbase + (size_t)k0 * HDIM, (uint32_t)((row16 + 16 * n) * HDIM + col16) * 2u);
      } else if (n < K_CH + V_CH) {
        const int i = n - K_CH;
        vr[i] = ld_u4(vbase + k0, (uint32_t)((v_d + 32 * i) * a.mp + v_kc) * 2u);
      } else {
        const int i = n - K_CH - V_CH;
        const int jn = jg00 + k0 + 128;  // first new band row of the tile at k0
        rr[i] = ld_u4(rbase, (uint32_t)(min(max(jn + row16 + 16 * i, 0), prows - 1) * HDIM + col16) * 2u);
      }
    };
    constexpr int N_FETCH = K_CH + V_CH + R_NEW;
    auto fetch = [&](int k0) {
#pragma unroll
      for (int n = 0; n < N_FETCH; ++n) fetch_one(k0, n);
    };
    // Staging needs no masks on K or relK: scores of keys >= T are replaced by
    // -inf in the softmax whatever K holds, and band rows outside [0, prows)
    // (clamped loads of valid rows) only meet (query, key) pairs with a query or
    // key past the sequence end. V^T columns of keys >= T are zeroed: their P is
    // 0, but 0 * (stale data) need not be 0.
    auto stage = [&](int k0, int t) {
#pragma unroll
      for (int i = 0; i < K_CH; ++i) *reinterpret_cast<uint4*>(&sm.K[(row16 + 16 * i) * KLD + col16]) = kr[i];
#pragma unroll
      for (int i = 0; i < V_CH; ++i) *reinterpret_cast<uint4*>(&sm.V[(v_d + 32 * i) * VLD + v_kc]) = vr[i];
      if (t > 0) {  // new band rows 128..191 of tile t -> ring blocks (4,5) + 2t
#pragma unroll
        for (int i = 0; i < R_NEW; ++i) {
          const int r = 128 + row16 + 16 * i;
          *reinterpret_cast<uint4*>(&sm.R[((((r >> 5) + 2 * t) % 6) * 32 + (r & 31)) * KLD + col16]) = rr[i];
        }
      }
      if (k0 + BKV > T) {  // the sequence's last tile (uniform branch)
        const int e0 = max(T - (k0 + v_kc), 0);  // valid keys of this thread's 8-key chunk
#pragma unroll
        for (int i = 0; i < V_CH; ++i)
#pragma nounroll
          for (int e = e0; e < 8; ++e) sm.V[(v_d + 32 * i) * VLD + v_kc + e] = (half)0.0f;
      }
    };

    const int rb0 = 96 - 32 * qg;  // first band row of this wave (3 ring blocks)
    fetch(k_begin);
    int t = 0;
    for (int k0 = k_begin; k0 < k_end; k0 += BKV, ++t) {
#pragma unroll
      for (int db = 0; db < 4; ++db) pin_acc(o[db]);
      stage(k0, t);
      __syncthreads();
#pragma unroll
      for (int db = 0; db < 4; ++db) pin_acc(o[db]);
      // The next tile's loads are issued two per step of the MFMA loop below
      // (the last tile re-reads its own valid addresses, so no branch is needed).
      const int k_next = k0 + BKV < k_end ? k0 + BKV : k0;

      // ---- content scores S^T (two 32-key blocks x 32 queries) and the position
      // band relK[j] . Qv^T over the wave's 96 band rows: five independent MFMA
      // chains, interleaved so they overlap in the pipeline
      floatx16 s0, s1, bd0, bd1, bd2;
#pragma unroll
      for (int v = 0; v < 16; ++v) s0[v] = s1[v] = bd0[v] = bd1[v] = bd2[v] = 0.0f;
      const int pb = (rb0 >> 5) + 2 * t;
      const int pb0 = pb % 6, pb1 = (pb + 1) % 6, pb2 = (pb + 2) % 6;  // ring blocks
      // Fragment reads run one 16-dim step ahead of the MFMAs (two register
      // sets); scheduling barriers keep the compiler from pulling them back
      // next to their MFMAs.
      half8 fr[2][5];
      auto frag_load = [&](int st, half8* f) {
        f[0] = ld_half8(&sm.K[l32 * KLD + 16 * st + 8 * lhi]);
        f[1] = ld_half8(&sm.K[(32 + l32) * KLD + 16 * st + 8 * lhi]);
        f[2] = ld_half8(&sm.R[(pb0 * 32 + l32) * KLD + 16 * st + 8 * lhi]);
        f[3] = ld_half8(&sm.R[(pb1 * 32 + l32) * KLD + 16 * st + 8 * lhi]);
        f[4] = ld_half8(&sm.R[(pb2 * 32 + l32) * KLD + 16 * st + 8 * lhi]);
      };
      frag_load(0, fr[0]);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        if (st < 7) frag_load(st + 1, fr[(st + 1) & 1]);
        if (2 * st < N_FETCH) fetch_one(k_next, 2 * st);
        if (2 * st + 1 < N_FETCH) fetch_one(k_next, 2 * st + 1);
        __builtin_amdgcn_sched_barrier(0);
        const half8* f = fr[st & 1];
        s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[0], quf[st], s0, 0, 0, 0);
        bd0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[2], qvf[st], bd0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[1], quf[st], s1, 0, 0, 0);
        bd1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[3], qvf[st], bd1, 0, 0, 0);
        bd2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[4], qvf[st], bd2, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const floatx4 w0 = {bd0[4 * g], bd0[4 * g + 1], bd0[4 * g + 2], bd0[4 * g + 3]};
        const floatx4 w1 = {bd1[4 * g], bd1[4 * g + 1], bd1[4 * g + 2], bd1[4 * g + 3]};
        const floatx4 w2 = {bd2[4 * g], bd2[4 * g + 1], bd2[4 * g + 2], bd2[4 * g + 3]};
        *reinterpret_cast<floatx4*>(&ps[l32 * PLD + 8 * g + 4 * lhi]) = w0;
        *reinterpret_cast<floatx4*>(&ps[l32 * PLD + 32 + 8 * g + 4 * lhi]) = w1;
        *reinterpret_cast<floatx4*>(&ps[l32 * PLD + 64 + 8 * g + 4 * lhi]) = w2;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // ---- rel-shift (diagonal read), mask, online softmax (log2 domain)
#pragma unroll
      for (int db = 0; db < 4; ++db) pin_acc(o[db]);
      // The row max is taken right after the sums in the same block, where the
      // compiler can see its inputs are arithmetic results and needs no
      // NaN-quieting; the sequence's last tile masks keys >= T and redoes it.
      float mt = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int kk = 8 * (v >> 2) + 4 * lhi + (v & 3);  // key within a 32-key block
        s0[v] += ps[l32 * PLD + kk + 31 - l32];
        s1[v] += ps[l32 * PLD + 32 + kk + 31 - l32];
        mt = fmaxf(mt, fmaxf(s0[v], s1[v]));
      }
      if (k0 + BKV > T) {  // uniform branch
        mt = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int kk = 8 * (v >> 2) + 4 * lhi + (v & 3);
          if (k0 + kk >= T) s0[v] = -INFINITY;
          if (k0 + 32 + kk >= T) s1[v] = -INFINITY;
          mt = fmaxf(mt, fmaxf(s0[v], s1[v]));
        }
      }
      mt = halves_max(mt);
      // Lazy rescaling: exp2 is taken against a reference max m_run that is only
      // raised when a new score exceeds it by more than 8 (log2 units), so
      // p <= 256 and the output/sum rescale runs rarely. Softmax is invariant to
      // the reference, so this is exact up to rounding.
      if (__any(mt > m_run + 8.0f)) {
        const float m_new = fmaxf(m_run, mt);
        const float corr = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= corr;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          floatx16 x = o[db];
          pin_vgpr(x);
#pragma unroll
          for (int v = 0; v < 16; ++v) x[v] *= corr;
          pin_acc(x);
          o[db] = x;
        }
        m_run = m_new;
      }
      const float m_use = m_run == -INFINITY ? 0.0f : m_run;  // no valid key yet
      float ls = 0.0f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p0 = __builtin_amdgcn_exp2f(s0[v] - m_use);
        const float p1 = __builtin_amdgcn_exp2f(s1[v] - m_use);
        s0[v] = p0;
        s1[v] = p1;
        ls += p0 + p1;
      }
      l_run += halves_sum(ls);

      // ---- O^T (128 d x 32 q) += V^T . P^T over the tile's 64 keys
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          half8 pf;
#pragma unroll
          for (int e = 0; e < 8; ++e) pf[e] = (half)(kb ? s1[8 * st + e] : s0[8 * st + e]);
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            const half* vp = &sm.V[(32 * db + l32) * VLD + 32 * kb + 16 * st + 4 * lhi];
            const half4 lo = *reinterpret_cast<const half4*>(vp);
            const half4 hi = *reinterpret_cast<const half4*>(vp + 8);
            const half8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, o[db], 0, 0, 0);
          }
        }
#pragma unroll
      for (int db = 0; db < 4; ++db) pin_acc(o[db]);
      __syncthreads();
    }

    // ---- output: the normalised rows, or this key range's partial
    const int ql = 32 * qg + l32;
    if (!complete) {  // o unnormalised (relative to m_run), with its max and sum
      const size_t sh = (size_t)slot * HEADS + h;
      float* po = a.part_o + (sh * BQ + ql) * HDIM;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const floatx4 w4 = {o[db][4 * g], o[db][4 * g + 1], o[db][4 * g + 2], o[db][4 * g + 3]};
          *reinterpret_cast<floatx4*>(po + 32 * db + 8 * g + 4 * lhi) = w4;
        }
      if (lhi == 0) {
        float* pm = a.part_ml + (sh * BQ + ql) * 2;
        pm[0] = m_run;
        pm[1] = l_run;
      }
    } else if (q_lane < T) {
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
  }  // segments
}

// Combines the key-range partials of one (query tile, head): with weights
// w_s = 2^(m_s - max_s m_s), out = sum_s w_s o_s / sum_s w_s l_s, slots in
// order. A workgroup covers 8 queries of one (merge entry, head); thread t
// handles query 8 * (group % 16) + t / 32, dims 4 * (t % 32) .. +3, so a launch
// has 16 workgroups per (query tile, head) and each thread streams one float4
// per slot.
constexpr int MERGE_Q = 8;
// Combine S slots with every load issued before the first combine (the
// running max and the sums keep slot order).
template <int S>
__device__ inline void merge_slots(const float* part_o, const float* part_ml, size_t sh0, size_t sstride, int d,
                                   floatx4& o, float& l) {
  float2 ml[S];
  floatx4 v[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const size_t sh = sh0 + s * sstride;
    ml[s] = *reinterpret_cast<const float2*>(part_ml + sh * 2);
    v[s] = *reinterpret_cast<const floatx4*>(part_o + sh * HDIM + d);
  }
  float m = -INFINITY;
#pragma unroll
  for (int s = 0; s < S; ++s) m = fmaxf(m, ml[s].x);
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const float w = __builtin_amdgcn_exp2f(ml[s].x - m);
    l += w * ml[s].y;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] += w * v[s][e];
  }
}

__global__ void __launch_bounds__(256) attn_merge_kernel(const float* part_o, const float* part_ml,
                                                         const int4* merges, half* out) {
  const int h = blockIdx.x % HEADS;
  const int rest = blockIdx.x / HEADS;
  const int4 mg = merges[rest / (BQ / MERGE_Q)];
  const int q = (rest % (BQ / MERGE_Q)) * MERGE_Q + (threadIdx.x >> 5);
  const int d = (threadIdx.x & 31) * 4;
  if (q >= mg.w) return;
  floatx4 o = {0.0f, 0.0f, 0.0f, 0.0f};
  float l = 0.0f;
  const size_t sh0 = ((size_t)mg.x * HEADS + h) * BQ + q, sstride = (size_t)HEADS * BQ;
  switch (mg.y) {
    case 2: merge_slots<2>(part_o, part_ml, sh0, sstride, d, o, l); break;
    case 3: merge_slots<3>(part_o, part_ml, sh0, sstride, d, o, l); break;
    case 4: merge_slots<4>(part_o, part_ml, sh0, sstride, d, o, l); break;
    default: {
      float m = -INFINITY;
      for (int s = 0; s < mg.y; ++s) m = fmaxf(m, part_ml[(sh0 + s * sstride) * 2]);
      for (int s = 0; s < mg.y; ++s) {
        const size_t sh = sh0 + s * sstride;
        const float w = __builtin_amdgcn_exp2f(part_ml[sh * 2] - m);
        l += w * part_ml[sh * 2 + 1];
        const floatx4 v = *reinterpret_cast<const floatx4*>(part_o + sh * HDIM + d);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] += w * v[e];
      }
    }
  }
  const float inv = 1.0f / l;
  const half4 w4 = {(half)(o[0] * inv), (half)(o[1] * inv), (half)(o[2] * inv), (half)(o[3] * inv)};
  *reinterpret_cast<half4*>(out + (size_t)(mg.z + q) * HIDDEN + h * HDIM + d) = w4;
}

}  // namespace

int attention_lanes(int t) {
  static const int forced = [] {
    const char* e = getenv("BARK_HIP_ATTN_LANES");
    return e ? atoi(e) : 0;
  }();
  // 32 lanes x 8 heads = one workgroup per CU of a 256-CU device
  const int units = ((t + BQ - 1) / BQ) * ((t + BKV - 1) / BKV);
  return std::max(1, std::min(forced > 0 ? forced : 32, units));
}

void rel_attention(const AttnArgs& a, hipStream_t stream) {
  BARK_REQUIRE(a.ntiles > 0 && a.tiles && a.nlanes > 0 && a.lanes, "rel_attention: no work segments");
  BARK_REQUIRE(a.mp % 64 == 0 && a.pp >= 2 * a.tc - 1, "rel_attention: bad buffer shape");
  BARK_REQUIRE((long long)a.mp * HDIM < (1ll << 31) && (long long)a.pp * HDIM < (1ll << 31),
               "rel_attention: per-head blocks must stay below 2^31 elements");
  static_assert(sizeof(Smem) <= 160 * 1024, "LDS budget");
  static_assert(K_CH * NT * 8 == BKV * HDIM && V_CH * NT * 8 == HDIM * BKV && R_NEW * NT * 8 == 64 * HDIM &&
                    R_CH * NT * 8 == BAND * HDIM,
                "staging chunks must tile the K, V^T and relK tiles exactly");
  static bool attr = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(rel_attn_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, sizeof(Smem)) == hipSuccess;
  }();
  BARK_REQUIRE(attr, "rel_attention: cannot reserve LDS");
  BARK_REQUIRE(a.nmerges == 0 || (a.merges && a.part_o && a.part_ml), "rel_attention: missing partial buffers");
  BARK_LAUNCH(rel_attn_kernel, dim3(a.nlanes * HEADS), dim3(NT), sizeof(Smem), stream, a);
  BARK_HIP_CHECK(hipGetLastError());
}

void rel_attention_merge(const AttnArgs& a, hipStream_t stream) {
  if (a.nmerges == 0) return;
  BARK_REQUIRE(a.merges && a.part_o && a.part_ml, "rel_attention_merge: missing partial buffers");
  BARK_LAUNCH(attn_merge_kernel, dim3(a.nmerges * HEADS * (BQ / MERGE_Q)), dim3(256), 0, stream, a.part_o, a.part_ml,
                     a.merges, a.out);
  BARK_HIP_CHECK(hipGetLastError());
}

// scale * log2(e) applied to q+u and q+v by the qkv epilogue
float attention_q_scale() { return (1.0f / sqrtf((float)HDIM)) * 1.4426950408889634f; }

}  // namespace bark
