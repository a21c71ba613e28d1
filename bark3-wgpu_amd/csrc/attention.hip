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

// Buffer-resource loads: an SGPR descriptor over [base, base + bytes) plus a
// 32-bit lane offset and a uniform offset, so a load needs one address VGPR.
// Offsets at or past the end read as zero.
__device__ inline __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ inline uint4 buffer_u4(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, uint32_t uniform_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)lane_off, (int)uniform_off, 0));
}

// LDS (address space 3) view of a workgroup-memory pointer: 32 bits, so it can
// sit in one vector register
typedef __attribute__((address_space(3))) float lds_float;
__device__ inline lds_float* to_lds(float* p) { return (lds_float*)p; }

// 16 bytes at base + byte offset off (a uniform base and a 32-bit lane offset)
__device__ inline uint4 ld_u4(const half* base, uint32_t off) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + off);
}

// A key-range partial of a query tile: the rows normalised by their own sum,
// o / l, in f16, and (m, l) in f32 (o is relative to the reference max m).
// Four 16-byte stores per lane per 32 rows of o (lane: query ql, dims
// 32 db + 8 g + 4 lhi .. + 3).
__device__ inline void write_partial(const AttnArgs& a, size_t sh, int bq, int ql, int lhi, const floatx16 (&o)[4],
                                     float m, float l) {
  const float inv = 1.0f / l;
  half* po = a.part_o + (sh * bq + ql) * HDIM;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const half4 w4 = {(half)(o[db][4 * g] * inv), (half)(o[db][4 * g + 1] * inv), (half)(o[db][4 * g + 2] * inv),
                        (half)(o[db][4 * g + 3] * inv)};
      *reinterpret_cast<half4*>(po + 32 * db + 8 * g + 4 * lhi) = w4;
    }
  if (lhi == 0) *reinterpret_cast<float2*>(a.part_ml + (sh * bq + ql) * 2) = make_float2(m, l);
}

// The normalised output rows of a complete query tile (lane: query q, dims as
// above), f16 into the heads-flat (rows, 1024) output.
__device__ inline void write_rows(const AttnArgs& a, size_t row, int h, int lhi, const floatx16 (&o)[4], float l) {
  const float inv = 1.0f / l;
  half* orow = a.out + row * HIDDEN + h * HDIM;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const half4 w4 = {(half)(o[db][4 * g] * inv), (half)(o[db][4 * g + 1] * inv), (half)(o[db][4 * g + 2] * inv),
                        (half)(o[db][4 * g + 3] * inv)};
      *reinterpret_cast<half4*>(orow + 32 * db + 8 * g + 4 * lhi) = w4;
    }
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
    if (!complete)
      write_partial(a, (size_t)slot * HEADS + h, BQ, ql, lhi, o, m_run, l_run);
    else if (q_lane < T)
      write_rows(a, (size_t)(start + q_lane), h, lhi, o, l_run);
  }  // segments
}

// Combines the key-range partials of one (query tile, head): with weights
// w_s = l_s 2^(m_s - max_s m_s), out = sum_s w_s (o_s / l_s) / sum_s w_s, slots
// in order. A workgroup covers 8 queries of one (merge entry, head); thread t
// handles query 8 * (group % (bq / 8)) + t / 32, dims 4 * (t % 32) .. +3, so a
// launch has bq / 8 workgroups per (query tile of bq queries, head) and each
// thread streams 8 bytes of o per slot.
constexpr int MERGE_Q = 8;
// Combine S slots with every load issued before the first combine (the
// running max and the sums keep slot order).
template <int S>
__device__ inline void merge_slots(const half* part_o, const float* part_ml, size_t sh0, size_t sstride, int d,
                                   floatx4& o, float& l) {
  float2 ml[S];
  half4 v[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const size_t sh = sh0 + s * sstride;
    ml[s] = *reinterpret_cast<const float2*>(part_ml + sh * 2);
    v[s] = *reinterpret_cast<const half4*>(part_o + sh * HDIM + d);
  }
  float m = -INFINITY;
#pragma unroll
  for (int s = 0; s < S; ++s) m = fmaxf(m, ml[s].x);
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const float w = ml[s].y * __builtin_amdgcn_exp2f(ml[s].x - m);
    l += w;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] += w * (float)v[s][e];
  }
}

__global__ void __launch_bounds__(256) attn_merge_kernel(const half* part_o, const float* part_ml,
                                                         const int4* merges, half* out, int bq) {
  const int h = blockIdx.x % HEADS;
  const int rest = blockIdx.x / HEADS;
  const int4 mg = merges[rest / (bq / MERGE_Q)];
  const int q = (rest % (bq / MERGE_Q)) * MERGE_Q + (threadIdx.x >> 5);
  const int d = (threadIdx.x & 31) * 4;
  if (q >= mg.w) return;
  floatx4 o = {0.0f, 0.0f, 0.0f, 0.0f};
  float l = 0.0f;
  const size_t sh0 = ((size_t)mg.x * HEADS + h) * bq + q, sstride = (size_t)HEADS * bq;
  switch (mg.y) {
    case 2: merge_slots<2>(part_o, part_ml, sh0, sstride, d, o, l); break;
    case 3: merge_slots<3>(part_o, part_ml, sh0, sstride, d, o, l); break;
    case 4: merge_slots<4>(part_o, part_ml, sh0, sstride, d, o, l); break;
    case 5: merge_slots<5>(part_o, part_ml, sh0, sstride, d, o, l); break;
    default: {
      float m = -INFINITY;
      for (int s = 0; s < mg.y; ++s) m = fmaxf(m, part_ml[(sh0 + s * sstride) * 2]);
      for (int s = 0; s < mg.y; ++s) {
        const size_t sh = sh0 + s * sstride;
        const float w = part_ml[sh * 2 + 1] * __builtin_amdgcn_exp2f(part_ml[sh * 2] - m);
        l += w;
        const half4 v = *reinterpret_cast<const half4*>(part_o + sh * HDIM + d);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] += w * (float)v[e];
      }
    }
  }
  const float inv = 1.0f / l;
  const half4 w4 = {(half)(o[0] * inv), (half)(o[1] * inv), (half)(o[2] * inv), (half)(o[3] * inv)};
  *reinterpret_cast<half4*>(out + (size_t)(mg.z + q) * HIDDEN + h * HDIM + d) = w4;
}

// ---------------------------------------------------------------------------
// Wide kernel (the default): 256 queries of one (sequence, head) per
// workgroup, 8 waves of 32 queries each, two waves per SIMD. A 64-key tile of
// K, V^T and the relK band is staged once for all eight waves, and every wave
// walks it in two 32-key sub-steps.
//
// Position band without recomputation: for a wave's 32 queries, the keys of
// sub-step sigma touch relative-position rows in two consecutive 32-row band
// blocks, b = sigma + 7 - qg and b + 1, and sub-step sigma + 1 needs blocks
// b + 1 and b + 2. So each sub-step computes ONE new block X = relK[block] .
// Qv^T (8 MFMAs, the same work as the content scores) and reuses the previous
// one. Row r of X in query lane l belongs to key (r + l + 1) & 31: of this
// sub-step when r + l + 1 < 32 (the "lower" part), of the next sub-step
// otherwise (the "upper" part, where X is the previous block). The band
// scratch is indexed by key, [query lane][32 keys]: the lower part is written
// before the scores read it back, the upper part after, for the next sub-step;
// the two parts fill complementary keys of every lane. The first sub-step of a
// segment computes its previous block's upper part too.
//
// Both waves of a SIMD run freely (their phases interleave by themselves):
// an explicit ping-pong of two wave groups over six barrier-delimited slots
// per tile measured slower, since the per-slot chains are bound by LDS
// fragment latency and the LDS / VALU work, not by missing MFMA overlap. The
// next tile's K, V^T and two new relK blocks are loaded into registers during
// the current tile's score MFMAs and staged after the tile's closing barrier.
//
// V^T is staged with the keys of every 16-key group in the order
// 0-3, 8-11, 4-7, 12-15, which is the P.V MFMA's key order for the exp'd
// scores as they sit in the score accumulators; so a lane reads its 8 keys of
// a V^T fragment as one 16-byte load.
constexpr int BQW = 256;
constexpr int NTW = 512;
constexpr int RBLK = 10;    // relK ring blocks of 32 rows: (BQW + BKV) / 32
constexpr int PLDW = 36;    // floats per query row of a wave's band scratch (32 used)
constexpr int KW_CH = BKV * HDIM / 8 / NTW;        // staging chunks per thread (512 threads)
constexpr int VW_CH = HDIM * BKV / 8 / NTW;
constexpr int RW_CH = RBLK * 32 * HDIM / 8 / NTW;

struct SmemW {
  half K[BKV * KLD];
  half V[HDIM * VLD];
  half R[RBLK * 32 * KLD];
  float P[8][32 * PLDW + 64];  // per wave: [32 query lanes][PLDW], then 64 junk floats
};

// V^T chunk of 8 keys (k0 + kc .. + 7 of d row `row`) into LDS in the P.V key
// order, keys >= T zeroed (0 * stale data need not be 0).
__device__ inline void stage_vt(half* V, int row, int kc, uint4 x, int valid) {
  if (valid < 8) {
    uint32_t* w = reinterpret_cast<uint32_t*>(&x);
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] &= (2 * e + 1 < valid ? 0xffff0000u : 0u) | (2 * e < valid ? 0xffffu : 0u);
  }
  half* p = V + row * VLD + (kc & ~15) + 4 * ((kc >> 3) & 1);
  *reinterpret_cast<uint2*>(p) = make_uint2(x.x, x.y);
  *reinterpret_cast<uint2*>(p + 8) = make_uint2(x.z, x.w);
}

__global__ void __launch_bounds__(NTW) rel_attn_wide_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  SmemW& sm = *reinterpret_cast<SmemW*>(smem_raw);

  // block b runs on XCD b % 8: head b % 8 keeps a head's tiles on one L2
  const int h = blockIdx.x % HEADS;
  const int wl = blockIdx.x / HEADS;
  const int tid = threadIdx.x, lane = tid & 63;
  const int qg = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave = query group
  const int l32 = lane & 31, lhi = lane >> 5;
  const int seg_end = a.lanes[wl + 1];
  for (int slot = a.lanes[wl]; slot < seg_end; ++slot) {
    const int4 tile = a.tiles[slot];
    const int start = tile.x, T = tile.y, q0 = tile.z;
    const int k_begin = (tile.w & 0xffff) * BKV, k_end = min(T, (tile.w >> 16) * BKV);
    const bool complete = k_begin == 0 && k_end == T;
    const int q_lane = q0 + 32 * qg + l32;
    const int prows = 2 * a.tc - 1;

    half8 quf[8], qvf[8];  // B operands: lane holds query q_lane, dims 16 s + 8 lhi .. + 7
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
    // relK ring: tile-relative band block b (32 rows from row jg00 + k_begin +
    // 32 b) lives in ring slot b % RBLK; tile t reads blocks 2t + 1 .. 2t + 9
    // (and 0 .. 7 for the first sub-step's previous blocks).
    const int jg00 = a.tc - 1 - (q0 + BQW - 1);
    auto rk_row = [&](int b, int r) {  // relK row r of band block b (clamped into the table)
      return rbase + (size_t)min(max(jg00 + k_begin + 32 * b + r, 0), prows - 1) * HDIM;
    };
    auto rk_off = [&](int b, int r) {  // the same as a byte offset from rbase (a head's block < 2^31)
      return (uint32_t)min(max(jg00 + k_begin + 32 * b + r, 0), prows - 1) * (uint32_t)(HDIM * 2);
    };

    // ---- segment prologue (all 512 threads): the ring's first ten blocks and
    // the first tile's K and V^T. Every load is issued before the first LDS
    // store, so the prologue waits for memory once (a load-store loop waited
    // once per pair of ring chunks).
    {
      const int col16 = (tid & 15) * 8, row32 = tid >> 4;
      const int vd = tid >> 3, kc = (tid & 7) * 8;
      uint4 pr[RW_CH], pk[KW_CH], pv[VW_CH];
#pragma unroll
      for (int i = 0; i < RW_CH; ++i) pr[i] = *reinterpret_cast<const uint4*>(rk_row(i, row32) + col16);
#pragma unroll
      for (int i = 0; i < KW_CH; ++i)
        pk[i] = ld_u4(kbase + (size_t)k_begin * HDIM, (uint32_t)((row32 + 32 * i) * HDIM + col16) * 2u);
#pragma unroll
      for (int i = 0; i < VW_CH; ++i) pv[i] = ld_u4(vbase + k_begin, (uint32_t)((vd + 64 * i) * a.mp + kc) * 2u);
#pragma unroll
      for (int i = 0; i < RW_CH; ++i) *reinterpret_cast<uint4*>(&sm.R[(32 * i + row32) * KLD + col16]) = pr[i];
#pragma unroll
      for (int i = 0; i < KW_CH; ++i) *reinterpret_cast<uint4*>(&sm.K[(row32 + 32 * i) * KLD + col16]) = pk[i];
#pragma unroll
      for (int i = 0; i < VW_CH; ++i) stage_vt(sm.V, vd + 64 * i, kc, pv[i], T - (k_begin + kc));
    }
    __syncthreads();

    // Band scratch of this wave, [query lane][key]. A value for key
    // (rho + e) & 31 of lane l32, e = l32 + 1 + 4 lhi, goes to pl[rho] when
    // rho + e < 32 (this sub-step) and to (pl - 32)[rho] otherwise (the next
    // one); a lane whose value belongs to the other part stores it to the junk
    // area instead (a per-lane address select, no branch).
    float* const pw = sm.P[qg];
    const int e_lane = l32 + 1 + 4 * lhi;
    lds_float* const pl = to_lds(pw + l32 * PLDW + e_lane);
    lds_float* const pj = to_lds(pw + 32 * PLDW + l32);
    // The two bases pass through an empty asm at every call, so the compiler
    // selects per store (one v_cndmask against a hoisted lane mask) instead of
    // keeping 32 selected addresses live across the loop.
    auto write_lower = [&](const floatx16& x) {
      lds_float *b = pl, *j = pj;
      asm volatile("" : "+v"(b), "+v"(j));
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rho = 8 * (v >> 2) + (v & 3);
        (rho + e_lane < 32 ? b : j)[rho] = x[v];
      }
    };
    // (the same condition as write_lower with the operands swapped: the two
    // share one set of 16 lane masks, which otherwise fill 64 SGPRs)
    auto write_upper = [&](const floatx16& x) {
      lds_float *b = pl - 32, *j = pj;
      asm volatile("" : "+v"(b), "+v"(j));
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rho = 8 * (v >> 2) + (v & 3);
        (rho + e_lane < 32 ? j : b)[rho] = x[v];
      }
    };
    auto wave_sync = [] {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // acc = A . B^T over the 128 dims: A rows from LDS (lane row l32, dims
    // 16 st + 8 lhi), B = the wave's query fragments. Fragment reads run one
    // step ahead of the MFMAs and no further (a compiler memory barrier plus a
    // scheduling barrier per step): hoisting them all would hold 32-64 more
    // registers.
    auto mfma_rows = [&](const half* ap, const half8 (&bf)[8], floatx16& acc) {
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
      half8 f[2];
      f[0] = ld_half8(ap);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        if (st < 7) f[(st + 1) & 1] = ld_half8(ap + 16 * (st + 1));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[st & 1], bf[st], acc, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // X = relK[band block b] . Qv^T (32 band rows x this wave's 32 queries)
    auto band_block = [&](int b, floatx16& x) {
      mfma_rows(&sm.R[((b % RBLK) * 32 + l32) * KLD + 8 * lhi], qvf, x);
    };
    // scores of sub-step sigma (keys 32 ss .. + 31 of the staged tile): the new
    // band block into x, the content S^T = K . Qu^T into s
    // The pins (empty asm on the results) keep each slot's MFMAs in that slot:
    // MFMAs are pure computations, and the compiler would otherwise sink them
    // past the barrier next to their consumers in the following slot.
    // The lower part of the band block goes to the scratch here, between the
    // band and the content MFMAs (which overlap the stores).
    // The band and content chains are independent: interleaved, each step has
    // two MFMAs to cover the next step's two fragment reads.
    auto scores = [&](int sigma, int ss, floatx16& x, floatx16& s) {
      const half* rp = &sm.R[(((sigma + 8 - qg) % RBLK) * 32 + l32) * KLD + 8 * lhi];
      const half* kp = &sm.K[(32 * ss + l32) * KLD + 8 * lhi];
#pragma unroll
      for (int v = 0; v < 16; ++v) x[v] = s[v] = 0.0f;
      half8 fr[2], fk[2];
      fr[0] = ld_half8(rp);
      fk[0] = ld_half8(kp);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        if (st < 7) {
          fr[(st + 1) & 1] = ld_half8(rp + 16 * (st + 1));
          fk[(st + 1) & 1] = ld_half8(kp + 16 * (st + 1));
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        x = __builtin_amdgcn_mfma_f32_32x32x16_f16(fr[st & 1], qvf[st], x, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(fk[st & 1], quf[st], s, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      pin_vgpr(x);
      pin_vgpr(s);
      write_lower(x);
    };
    // rel-shift through the band scratch, mask, online softmax (log2 domain);
    // the exp'd scores as the two 16-key B operands of P.V. The block's upper
    // part is stored later (write_upper), once these reads are done.
    auto softmax = [&](int kw, floatx16& s, half8& p0, half8& p1) {
      wave_sync();
      float mt = -INFINITY;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const floatx4 b4 = *reinterpret_cast<const floatx4*>(&pw[l32 * PLDW + 8 * g + 4 * lhi]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s[4 * g + e] += b4[e];
          mt = fmaxf(mt, s[4 * g + e]);
        }
      }
      if (kw + 32 > T) {  // uniform branch: the sequence's last keys
        mt = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int kk = 8 * (v >> 2) + 4 * lhi + (v & 3);
          if (kw + kk >= T) s[v] = -INFINITY;
          mt = fmaxf(mt, s[v]);
        }
      }
      mt = halves_max(mt);
      // lazy rescaling (threshold 8 in log2 units), as in the four-wave kernel
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
      const float m_use = m_run == -INFINITY ? 0.0f : m_run;
      float ls = 0.0f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = __builtin_amdgcn_exp2f(s[v] - m_use);
        s[v] = p;
        ls += p;
      }
      l_run += halves_sum(ls);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p0[e] = (half)s[e];
        p1[e] = (half)s[8 + e];
      }
      pin_vgpr(p0);
      pin_vgpr(p1);
    };
    // O^T (128 d x 32 q) += V^T . P^T over the sub-step's 32 keys
    auto pv = [&](int ss, const half8& p0, const half8& p1) {
      const half* vp = &sm.V[l32 * VLD + 32 * ss + 8 * lhi];
      half8 f[2];
      f[0] = ld_half8(vp);
#pragma unroll
      for (int i = 0; i < 8; ++i) {  // i = 4 st + db
        if (i < 7) f[(i + 1) & 1] = ld_half8(vp + 32 * ((i + 1) & 3) * VLD + 16 * ((i + 1) >> 2));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        o[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i & 1], i >> 2 ? p1 : p0, o[i & 3], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) pin_vgpr(o[db]);
    };
    auto first_upper = [&] {  // previous block of the segment's first sub-step
      floatx16 x0;
      band_block(7 - qg, x0);
      pin_vgpr(x0);
      write_upper(x0);
    };

    // Per-tile staging by all 512 threads: K rows and relK block rows (16
    // chunks of 8 halves per row), V^T d rows (8 chunks of 8 keys per row).
    const int col16 = (tid & 15) * 8, row32 = tid >> 4;  // + 32 i
    const int vd = tid >> 3, kc = (tid & 7) * 8;         // + 64 i
    // the head's K, V^T and relK blocks as buffer resources (each < 2^31 bytes)
    const __amdgpu_buffer_rsrc_t kr = buffer_rsrc(kbase, (uint32_t)((a.mp - start) * HDIM * 2));
    const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(vbase, (uint32_t)((HDIM * a.mp - start) * 2));
    const __amdgpu_buffer_rsrc_t rr = buffer_rsrc(rbase, (uint32_t)(prows * HDIM * 2));
    const uint32_t koff = (uint32_t)(row32 * HDIM + col16) * 2u, voff = (uint32_t)(vd * a.mp + kc) * 2u;
    // the next tile into registers: K rows, V^T columns, relK blocks 2t + 10 and 2t + 11
    uint4 nk[KW_CH], nv[VW_CH], nr[2];
    auto fetch_one = [&](int k_next, int t, int n) {
      if (n < KW_CH) {
        nk[n] = buffer_u4(kr, koff, (uint32_t)((k_next + 32 * n) * HDIM * 2));
      } else if (n < KW_CH + VW_CH) {
        const int i = n - KW_CH;
        nv[i] = buffer_u4(vr, voff, (uint32_t)(k_next * 2 + i * 64 * a.mp * 2));
      } else {
        const int i = n - KW_CH - VW_CH;
        nr[i] = buffer_u4(rr, rk_off(2 * t + 10 + i, row32) + col16 * 2u, 0);
      }
    };
    static_assert(KW_CH + VW_CH + 2 == 6, "six prefetch loads per tile, three per sub-step");

    floatx16 x, s;
    half8 p0, p1;
    int t = 0;
    for (int k0 = k_begin; k0 < k_end; k0 += BKV, ++t) {
      if (t > 0) {  // stage the prefetched tile (the previous tile ended with a barrier)
#pragma unroll
        for (int i = 0; i < KW_CH; ++i) *reinterpret_cast<uint4*>(&sm.K[(row32 + 32 * i) * KLD + col16]) = nk[i];
#pragma unroll
        for (int i = 0; i < VW_CH; ++i) stage_vt(sm.V, vd + 64 * i, kc, nv[i], T - (k0 + kc));
#pragma unroll
        for (int i = 0; i < 2; ++i)
          *reinterpret_cast<uint4*>(&sm.R[(((2 * t + 8 + i) % RBLK) * 32 + row32) * KLD + col16]) = nr[i];
        __syncthreads();
      }
      const int k_next = __builtin_amdgcn_readfirstlane(k0 + BKV < k_end ? k0 + BKV : k0);
      if (t == 0) first_upper();
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        const int kw = k0 + 32 * ss;
        if (kw >= T) break;  // uniform: past the sequence end
        scores(2 * t + ss, ss, x, s);
#pragma unroll
        for (int n = 0; n < 3; ++n) fetch_one(k_next, t, 3 * ss + n);
        softmax(kw, s, p0, p1);
        write_upper(x);
        pv(ss, p0, p1);
      }
      __syncthreads();
    }

    const int ql = 32 * qg + l32;
    if (!complete)
      write_partial(a, (size_t)slot * HEADS + h, BQW, ql, lhi, o, m_run, l_run);
    else if (q_lane < T)
      write_rows(a, (size_t)(start + q_lane), h, lhi, o, l_run);
  }  // segments
}

// 4 selects the four-wave, 128-query kernel; anything else the wide one
int attention_kernel_waves() {
  static const int w = [] {
    const char* e = getenv("BARK_HIP_ATTN_WAVES");
    return e && atoi(e) == 4 ? 4 : 8;
  }();
  return w;
}

}  // namespace

int attention_query_tile() { return attention_kernel_waves() == 4 ? BQ : BQW; }

int attention_lanes(int t) {
  static const int forced = [] {
    const char* e = getenv("BARK_HIP_ATTN_LANES");
    return e ? atoi(e) : 0;
  }();
  // 32 lanes x 8 heads = one workgroup per CU of a 256-CU device
  const int bq = attention_query_tile();
  const int units = ((t + bq - 1) / bq) * ((t + BKV - 1) / BKV);
  return std::max(1, std::min(forced > 0 ? forced : 32, units));
}

void rel_attention(const AttnArgs& a, hipStream_t stream) {
  BARK_REQUIRE(a.ntiles > 0 && a.tiles && a.nlanes > 0 && a.lanes, "rel_attention: no work segments");
  BARK_REQUIRE(a.mp % 64 == 0 && a.pp >= 2 * a.tc - 1, "rel_attention: bad buffer shape");
  BARK_REQUIRE((long long)a.mp * HDIM < (1ll << 31) && (long long)a.pp * HDIM < (1ll << 31),
               "rel_attention: per-head blocks must stay below 2^31 elements");
  BARK_REQUIRE(a.nmerges == 0 || (a.merges && a.part_o && a.part_ml), "rel_attention: missing partial buffers");
  if (attention_kernel_waves() == 4) {
    static_assert(sizeof(Smem) <= 160 * 1024, "LDS budget");
    static_assert(K_CH * NT * 8 == BKV * HDIM && V_CH * NT * 8 == HDIM * BKV && R_NEW * NT * 8 == 64 * HDIM &&
                      R_CH * NT * 8 == BAND * HDIM,
                  "staging chunks must tile the K, V^T and relK tiles exactly");
    static bool attr = [] {
      return hipFuncSetAttribute(reinterpret_cast<const void*>(rel_attn_kernel),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, sizeof(Smem)) == hipSuccess;
    }();
    BARK_REQUIRE(attr, "rel_attention: cannot reserve LDS");
    BARK_LAUNCH(rel_attn_kernel, dim3(a.nlanes * HEADS), dim3(NT), sizeof(Smem), stream, a);
  } else {
    static_assert(sizeof(SmemW) <= 160 * 1024, "LDS budget");
    static_assert(KW_CH * NTW * 8 == BKV * HDIM && VW_CH * NTW * 8 == HDIM * BKV &&
                      RW_CH * NTW * 8 == RBLK * 32 * HDIM && RBLK * 32 == BQW + BKV && NTW * 8 == 32 * HDIM,
                  "staging chunks must tile the K, V^T and relK tiles exactly");
    static bool attr = [] {
      return hipFuncSetAttribute(reinterpret_cast<const void*>(rel_attn_wide_kernel),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, sizeof(SmemW)) == hipSuccess;
    }();
    BARK_REQUIRE(attr, "rel_attention: cannot reserve LDS");
    BARK_LAUNCH(rel_attn_wide_kernel, dim3(a.nlanes * HEADS), dim3(NTW), sizeof(SmemW), stream, a);
  }
  BARK_HIP_CHECK(hipGetLastError());
}

void rel_attention_merge(const AttnArgs& a, hipStream_t stream) {
  if (a.nmerges == 0) return;
  BARK_REQUIRE(a.merges && a.part_o && a.part_ml, "rel_attention_merge: missing partial buffers");
  const int bq = attention_query_tile();
  BARK_LAUNCH(attn_merge_kernel, dim3(a.nmerges * HEADS * (bq / MERGE_Q)), dim3(256), 0, stream, a.part_o,
              a.part_ml, a.merges, a.out, bq);
  BARK_HIP_CHECK(hipGetLastError());
}

// scale * log2(e) applied to q+u and q+v by the qkv epilogue
float attention_q_scale() { return (1.0f / sqrtf((float)HDIM)) * 1.4426950408889634f; }

}  // namespace bark
