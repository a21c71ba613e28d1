// GEMM for the encoder linears on gfx950 MFMA.
//
// C[m, n] = sum_k A[m, k] * W[n, k] with A f16 (activations) and W either f16
// or 4-bit codes with a per-output-row 16-entry f16 table (`W[n,k] =
// lut[n][code(n,k)]`). Accumulation is f32 on v_mfma_f32_32x32x16_f16.
//
// Reference: the WGSL `gemm_mix_bm64[_lb]` / `gemm_mix_8x4` family
// (src/encoder/gemm.rs:225-683) and the CPU `gemm` (src/cpu/gemm.rs:220-311)
// compute the same product with f32 activations. f16 levels are exact in the
// f16 MFMA operand, so dequantisation here is bit-exact; only the activation
// operand is rounded (to f16) and the accumulation order differs.
//
// Tiling: 256 threads = 4 waves in a 2x2 grid; workgroup tile BM x 128 with
// BK = 64; each wave owns a (BM/2) x 64 patch made of 32x32 MFMA blocks.
// A and B tiles are staged through LDS (double-buffered, rows padded by 16 B so
// the 16-byte fragment reads of 8 lanes hit disjoint banks). In LUT4 mode each
// thread owns one weight row for the whole kernel: its 16-entry f16 table sits
// in 8 VGPRs as low-byte and high-byte planes, and every k-tile it streams 16
// bytes of codes (32 weights) with one coalesced load and expands them with
// byte permutes (v_perm_b32) — no LDS lookups — into the f16 B tile, so every
// weight is expanded once per workgroup and reused by all BM rows.
//
// Code layouts: "plain" = two codes per byte, low nibble = even k (the
// reference's layout); "swizzled" = within each 4-byte group of 8 codes, byte i
// holds codes i (low nibble) and i+4 (high nibble), which the expansion turns
// into natural k order with half the permutes. Encoder weights are swizzled
// once at load.
#include <cstdlib>
#include <map>
#include <mutex>
#include <type_traits>
#include <utility>

#include "kernels.h"

namespace bark {
namespace {

constexpr int BN = 128;
constexpr int BK = 64;
constexpr int LDK = BK + 8;  // halves per LDS row (144 B)

struct GemmParams {
  const half* A;
  int lda;
  const half* W;
  const uint8_t* codes;
  const half* lut;
  int M, N, K;
  EpiArgs ea;
  int splits = 1;        // wide kernel: K chunks (blockIdx.z selects one); chunk s covers
                         // 256-k units [s*q + min(s, r), ...) of K/256 = q*splits + r
  size_t out_zstride = 0;  // wide kernel: elements between the splits' outputs
};

__device__ inline uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Row table as byte planes: L[q] holds the low bytes of entries 4q..4q+3,
// H[q] the high bytes. c4 is the constant 0x04040404; with OPQ it sits in a
// vector register (opaque to the compiler), so the select mask of lookup4 is
// one v_and_or_b32 (gfx950's three-operand encoding takes no 32-bit literal,
// and with two literals the compiler splits it into an AND and an OR): 23
// VALU instructions per 8 weights instead of 25, for one register, which
// kernels at the register limit do without (OPQ = false).
struct RowLut {
  uint32_t L[4], H[4];
  uint32_t c4;
};

template <bool OPQ = true>
__device__ inline RowLut load_row_lut(const half* lut_row) {
  const uint4 a = *reinterpret_cast<const uint4*>(lut_row);
  const uint4 b = *reinterpret_cast<const uint4*>(lut_row + 8);
  const uint32_t d[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  RowLut t;
  uint32_t c4 = 0x04040404u;
  if constexpr (OPQ) asm volatile("" : "+v"(c4));
  t.c4 = c4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    t.L[q] = perm(d[2 * q + 1], d[2 * q], 0x06040200u);
    t.H[q] = perm(d[2 * q + 1], d[2 * q], 0x07050301u);
  }
  return t;
}

// Four codes (one per byte of x, values 0..15) -> low and high bytes of their
// table entries.
__device__ inline void lookup4(uint32_t x, const RowLut& t, uint32_t& lo, uint32_t& hi) {
  const uint32_t s7 = x & 0x07070707u;
  const uint32_t la = perm(t.L[1], t.L[0], s7), lb = perm(t.L[3], t.L[2], s7);
  const uint32_t ha = perm(t.H[1], t.H[0], s7), hb = perm(t.H[3], t.H[2], s7);
  const uint32_t ms = ((x >> 1) & t.c4) | 0x03020100u;  // byte i: i, or i+4 if code >= 8
  lo = perm(lb, la, ms);
  hi = perm(hb, ha, ms);
}

// One u32 of codes (8 consecutive k) -> 8 f16 in natural k order.
template <bool SWZ>
__device__ inline uint4 expand8(uint32_t w, const RowLut& t) {
  uint32_t le, he, lo_, ho;
  lookup4(w & 0x0F0F0F0Fu, t, le, he);
  lookup4((w >> 4) & 0x0F0F0F0Fu, t, lo_, ho);
  if constexpr (SWZ) {  // le/he: k 0..3, lo_/ho: k 4..7
    return uint4{perm(he, le, 0x05010400u), perm(he, le, 0x07030602u), perm(ho, lo_, 0x05010400u),
                 perm(ho, lo_, 0x07030602u)};
  } else {  // le/he: k 0,2,4,6, lo_/ho: k 1,3,5,7
    const uint32_t e01 = perm(he, le, 0x05010400u), e23 = perm(he, le, 0x07030602u);
    const uint32_t o01 = perm(ho, lo_, 0x05010400u), o23 = perm(ho, lo_, 0x07030602u);
    return uint4{perm(o01, e01, 0x05040100u), perm(o01, e01, 0x07060302u), perm(o23, e23, 0x05040100u),
                 perm(o23, e23, 0x07060302u)};
  }
}

// bf16 -> f16 of 8 consecutive k (exact for |x| in the f16 normal range),
// stored in the k order 0, 2, 4, 6, 1, 3, 5, 7: the order expand8<true> gives
// a plain-layout code word (byte j = codes 2j, 2j + 1 read as codes j, j + 4).
// An MFMA sums the same products whatever the order of its operands' k, so
// bf16 activations staged this way meet plain 4-bit weights expanded with the
// swizzled layout's cheaper permutes; the conversion's placement is free.
__device__ inline half8 bf16x8_to_f16_eo(uint4 x) {
  const uint32_t w4[4] = {x.x, x.y, x.z, x.w};
  half8 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = (half)__uint_as_float(w4[e] << 16);
    v[4 + e] = (half)__uint_as_float(w4[e] & 0xffff0000u);
  }
  return v;
}

// f32 -> f16 after materialising the f32 value: the compiler may otherwise
// fuse a multiply with the conversion (one rounding) in some epilogue
// instantiations and not in others, which would make a row's f16 output
// depend on the tile it falls in.
__device__ inline half to_f16(float x) {
  asm volatile("" : "+v"(x));
  return (half)x;
}

__device__ inline float fast_sigmoid_mul(float a, float g) {
  return a * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

template <int EPI>
__device__ inline void store_one(const EpiArgs& ea, int r, int c, float v) {
  if constexpr (EPI == (int)Epi::StoreF32) {
    if (ea.bias) v += ea.bias[c];
    ea.out_f32[(size_t)r * ea.ldo + c] = v;
  } else if constexpr (EPI == (int)Epi::StoreF16) {
    if (ea.bias) v += ea.bias[c];
    ea.out_f16[(size_t)r * ea.ldo + c] = to_f16(v);
  } else if constexpr (EPI == (int)Epi::StoreBF16) {
    if (ea.bias) v += ea.bias[c];
    uint32_t u = __float_as_uint(v);
    u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even (finite inputs)
    reinterpret_cast<uint16_t*>(ea.out_f16)[(size_t)r * ea.ldo + c] = (uint16_t)(u >> 16);
  } else if constexpr (EPI == (int)Epi::Silu) {
    ea.out_f16[(size_t)r * ea.ldo + c] = to_f16(fast_sigmoid_mul(v, v));
  } else if constexpr (EPI == (int)Epi::Resid) {
    float* p = ea.out_f32 + (size_t)r * ea.ldo + c;
    *p = *p + ea.scale * v;
  } else if constexpr (EPI == (int)Epi::ResidHalf) {
    float* p = ea.out_f32 + (size_t)r * ea.ldo + c;
    *p = *p + 0.5f * v;
  } else if constexpr (EPI == (int)Epi::Qkv) {
    const int which = c >> 10, hd = c & 1023, h = hd >> 7, d = hd & 127;
    const size_t hr = ((size_t)h * ea.mp + r) * HDIM + d;
    if (which == 0) {
      ea.qu[hr] = to_f16((v + ea.bu[hd]) * ea.scale);
      ea.qv[hr] = to_f16((v + ea.bv[hd]) * ea.scale);
    } else if (which == 1) {
      ea.kh[hr] = to_f16(v);
    } else {
      ea.vt[((size_t)h * HDIM + d) * ea.mp + r] = to_f16(v);
    }
  } else if constexpr (EPI == (int)Epi::RelK) {
    const int h = c >> 7, d = c & 127;
    ea.rk[((size_t)h * ea.pp + r) * HDIM + d] = to_f16(v);
  } else if constexpr (EPI == (int)Epi::BiasReluF16) {
    v += ea.bias[c];
    ea.out_f16[(size_t)r * ea.ldo + c] = to_f16(v > 0.0f ? v : 0.0f);
  } else if constexpr (EPI == (int)Epi::FlattenReluF16) {
    v += ea.bias[c];
    const int t = r >> 4, m = r & 15;
    ea.out_f16[(size_t)t * ea.ldo + c * 16 + m] = to_f16(v > 0.0f ? v : 0.0f);
  }
}

template <int BM, bool LUT4, bool SWZ, bool ABF16, int EPI>
__global__ void __launch_bounds__(256) gemm_kernel(GemmParams p) {
  constexpr int WTM = BM / 2;       // wave tile rows
  constexpr int FM = WTM / 32;      // 32-row MFMA blocks per wave
  constexpr int FN = 2;             // 32-col MFMA blocks per wave (64 cols)
  constexpr int A_CH = BM * BK / 8 / 256;  // 16-byte chunks of A per thread
  constexpr int B_CH = BN * BK / 8 / 256;  // (f16 mode)

  __shared__ __attribute__((aligned(16))) half As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) half Bs[2][BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int l32 = lane & 31, lhi = lane >> 5;

  // Four register stages hold the k-tiles in flight from global memory: a
  // tile's loads are issued three iterations of MFMA work before its LDS
  // store, which covers HBM latency.
  struct Stage {
    uint4 a[A_CH];
    uint4 b[LUT4 ? 1 : B_CH];
  };
  Stage r0, r1, r2, r3;

  RowLut lut;  // this thread's weight row: n0 + tid/2
  if constexpr (LUT4) lut = load_row_lut(p.lut + (size_t)(n0 + (tid >> 1)) * 16);

  auto load_tiles = [&](int kt, Stage& st) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int ch = tid + 256 * i, row = ch >> 3, col = (ch & 7) * 8;
      st.a[i] = (m0 + row < p.M)
                    ? *reinterpret_cast<const uint4*>(p.A + (size_t)(m0 + row) * p.lda + k0 + col)
                    : uint4{0u, 0u, 0u, 0u};
    }
    if constexpr (LUT4) {
      const int row = tid >> 1, part = tid & 1;
      st.b[0] = *reinterpret_cast<const uint4*>(p.codes + (size_t)(n0 + row) * (p.K >> 1) +
                                                (k0 >> 1) + part * 16);
    } else {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int ch = tid + 256 * i, row = ch >> 3, col = (ch & 7) * 8;
        st.b[i] = *reinterpret_cast<const uint4*>(p.W + (size_t)(n0 + row) * p.K + k0 + col);
      }
    }
  };

  auto store_tiles = [&](int stage, const Stage& st) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int ch = tid + 256 * i, row = ch >> 3, col = (ch & 7) * 8;
      if constexpr (ABF16) {  // bf16 -> f16: exact for |x| in the f16 normal range
        const uint32_t w4[4] = {st.a[i].x, st.a[i].y, st.a[i].z, st.a[i].w};
        half8 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = (half)__uint_as_float(w4[e] << 16);
          v[2 * e + 1] = (half)__uint_as_float(w4[e] & 0xffff0000u);
        }
        st_half8(&As[stage][row * LDK + col], v);
      } else {
        *reinterpret_cast<uint4*>(&As[stage][row * LDK + col]) = st.a[i];
      }
    }
    if constexpr (LUT4) {
      const int row = tid >> 1, part = tid & 1;
      const uint32_t w4[4] = {st.b[0].x, st.b[0].y, st.b[0].z, st.b[0].w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<uint4*>(&Bs[stage][row * LDK + part * 32 + q * 8]) = expand8<SWZ>(w4[q], lut);
    } else {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int ch = tid + 256 * i, row = ch >> 3, col = (ch & 7) * 8;
        *reinterpret_cast<uint4*>(&Bs[stage][row * LDK + col]) = st.b[i];
      }
    }
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  auto compute = [&](int cur) {
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      half8 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = ld_half8(&As[cur][(wm * WTM + i * 32 + l32) * LDK + ks * 16 + lhi * 8]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = ld_half8(&Bs[cur][(wn * 64 + j * 32 + l32) * LDK + ks * 16 + lhi * 8]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  // One k-tile of MFMAs from LDS stage `cur`, fused with writing the next
  // k-tile (register stage `st`) into LDS stage `nxt`: each 16-k slice issues
  // its fragment reads, expands one code word of the next tile (VALU) and
  // stores it, and runs its MFMAs, so the matrix cores keep working while the
  // codes are expanded. Scheduler groups keep that order per slice.
  auto step = [&](int cur, int nxt, const Stage& st) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int ch = tid + 256 * i, row = ch >> 3, col = (ch & 7) * 8;
      if constexpr (ABF16) {
        const uint32_t w4[4] = {st.a[i].x, st.a[i].y, st.a[i].z, st.a[i].w};
        half8 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = (half)__uint_as_float(w4[e] << 16);
          v[2 * e + 1] = (half)__uint_as_float(w4[e] & 0xffff0000u);
        }
        st_half8(&As[nxt][row * LDK + col], v);
      } else {
        *reinterpret_cast<uint4*>(&As[nxt][row * LDK + col]) = st.a[i];
      }
    }
    const int brow = tid >> 1, bpart = tid & 1;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      half8 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = ld_half8(&As[cur][(wm * WTM + i * 32 + l32) * LDK + ks * 16 + lhi * 8]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = ld_half8(&Bs[cur][(wn * 64 + j * 32 + l32) * LDK + ks * 16 + lhi * 8]);
      if constexpr (LUT4) {
        const uint32_t w = ks == 0 ? st.b[0].x : ks == 1 ? st.b[0].y : ks == 2 ? st.b[0].z : st.b[0].w;
        const uint4 q = expand8<SWZ>(w, lut);
        *reinterpret_cast<uint4*>(&Bs[nxt][brow * LDK + bpart * 32 + ks * 8]) = q;
      } else {
#pragma unroll
        for (int i = ks * B_CH / 4; i < (ks + 1) * B_CH / 4; ++i) {
          const int ch = tid + 256 * i, row = ch >> 3, col = (ch & 7) * 8;
          *reinterpret_cast<uint4*>(&Bs[nxt][row * LDK + col]) = st.b[i];
        }
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
      constexpr int VPER = LUT4 ? (26 + FM * FN - 1) / (FM * FN) : 1;
      __builtin_amdgcn_sched_group_barrier(0x100, FM + FN, 0);
#pragma unroll
      for (int m = 0; m < FM * FN; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, VPER, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
    }
  };

  // K is a multiple of 4*BK: the loop runs in branch-free groups of four
  // k-tiles. At the top of each group LDS stage 0 holds tile kt and register
  // stages r1..r3 hold tiles kt+1..kt+3; each step computes one tile, stores the
  // next one into the other LDS stage and refills the register stage it freed.
  const int nk = p.K / BK;
  load_tiles(0, r0);
  load_tiles(1, r1);
  load_tiles(2, r2);
  load_tiles(3, r3);
  store_tiles(0, r0);
  __syncthreads();
  for (int kt = 0; kt + 4 < nk; kt += 4) {
    load_tiles(kt + 4, r0);
    step(0, 1, r1);
    __syncthreads();
    load_tiles(kt + 5, r1);
    step(1, 0, r2);
    __syncthreads();
    load_tiles(kt + 6, r2);
    step(0, 1, r3);
    __syncthreads();
    load_tiles(kt + 7, r3);
    step(1, 0, r0);
    __syncthreads();
  }
  step(0, 1, r1);
  __syncthreads();
  step(1, 0, r2);
  __syncthreads();
  step(0, 1, r3);
  __syncthreads();
  compute(1);

  // Epilogue. Accumulator element v of lane `lane` in block (i, j) is
  // row 8*(v/4) + 4*(lane/32) + v%4, column lane%32 of that 32x32 block.
  const EpiArgs& ea = p.ea;
  if constexpr (EPI == (int)Epi::Glu) {
    // W rows are interleaved so this wave's two column blocks hold the GLU
    // pair: block 0 = value half, block 1 = gate half of output column c.
    const int c = ((n0 + wn * 64) >> 1) + l32;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = m0 + wm * WTM + i * 32 + 8 * (v >> 2) + 4 * lhi + (v & 3);
        if (r >= p.M) continue;
        const float a = acc[i][0][v], g = acc[i][1][v];
        ea.out_f32[(size_t)r * ea.ldo + c] = fast_sigmoid_mul(a, g);
      }
  } else {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = m0 + wm * WTM + i * 32 + 8 * (v >> 2) + 4 * lhi + (v & 3);
          const int c = n0 + wn * 64 + j * 32 + l32;
          if (r < p.M) store_one<EPI>(ea, r, c, acc[i][j][v]);
        }
  }
}

// Epilogue of a (32*FM) x (32*NB) wave tile. Lane (l32, lhi) holds, for MFMA block (i, j), column
// nw + 32j + l32 and rows m0 + 32i + 8g + 4lhi + b of acc[i][j][4g + b].
// Column-dependent work (bias, head/dim split, output base) is done once
// per column; row offsets are compile-time multiples of the row stride; a
// tile inside M skips the per-row bound checks. bz selects the split-K slab.
template <int FM, int EPI, int NB = 2>
__device__ inline void tile_epilogue(floatx16 (&acc)[FM][NB], const GemmParams& p, int m0, int nw, int bz, int lane,
                                     int ib = 0, int ie = FM) {
  const int l32 = lane & 31, lhi = lane >> 5;
  EpiArgs ea = p.ea;
  if constexpr (EPI == (int)Epi::StoreF32) ea.out_f32 += bz * p.out_zstride;
  const int mrow = m0 + 4 * lhi;  // row of acc element v = 0 of block i = 0
  auto epilogue = [&](auto checked) {
  constexpr bool CHK = decltype(checked)::value;
  auto row_ok = [&](int rl) { return !CHK || mrow + rl < p.M; };  // rl = 32i + 8g + b
  if constexpr (EPI == (int)Epi::Glu) {
    static_assert(NB == 2, "GLU pairs need both column blocks of a wave");
    float* base = ea.out_f32 + (size_t)mrow * ea.ldo + (nw >> 1) + l32;
#pragma unroll
    for (int i = 0; i < FM; ++i) if (i >= ib && i < ie)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rl = 32 * i + 8 * (v >> 2) + (v & 3);
        if (row_ok(rl)) base[(size_t)rl * ea.ldo] = fast_sigmoid_mul(acc[i][0][v], acc[i][NB - 1][v]);
      }
  } else if constexpr (EPI == (int)Epi::Qkv) {
    const int region = __builtin_amdgcn_readfirstlane(nw >> 10);  // 0 q, 1 k, 2 v (wave-uniform)
    if (region == 2) {
      // V^T[h][d][r]: a lane's four consecutive rows are contiguous, one 8-byte store
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int hd = nw - 2048 + 32 * j + l32;  // h*128 + d
        half* vrow = ea.vt + (size_t)hd * ea.mp + mrow;
#pragma unroll
        for (int i = 0; i < FM; ++i) if (i >= ib && i < ie)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int rl = 32 * i + 8 * g;
            if (!CHK || mrow + rl + 3 < p.M) {
              const half4 w4 = {to_f16(acc[i][j][4 * g]), to_f16(acc[i][j][4 * g + 1]),
                                to_f16(acc[i][j][4 * g + 2]), to_f16(acc[i][j][4 * g + 3])};
              *reinterpret_cast<half4*>(vrow + rl) = w4;
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (mrow + rl + e < p.M) vrow[rl + e] = to_f16(acc[i][j][4 * g + e]);
            }
          }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int hd = (nw & 1023) + 32 * j + l32, h = hd >> 7, d = hd & 127;
        const size_t off = ((size_t)h * ea.mp + mrow) * HDIM + d;
        if (region == 0) {
          const float bu = ea.bu[hd], bv = ea.bv[hd];
          half* pu = ea.qu + off;
          half* pv = ea.qv + off;
#pragma unroll
          for (int i = 0; i < FM; ++i) if (i >= ib && i < ie)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int rl = 32 * i + 8 * (v >> 2) + (v & 3);
              if (row_ok(rl)) {
                pu[rl * HDIM] = to_f16((acc[i][j][v] + bu) * ea.scale);
                pv[rl * HDIM] = to_f16((acc[i][j][v] + bv) * ea.scale);
              }
            }
        } else {
          half* pk = ea.kh + off;
#pragma unroll
          for (int i = 0; i < FM; ++i) if (i >= ib && i < ie)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int rl = 32 * i + 8 * (v >> 2) + (v & 3);
              if (row_ok(rl)) pk[rl * HDIM] = to_f16(acc[i][j][v]);
            }
        }
      }
    }
  } else if constexpr (EPI == (int)Epi::RelK) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int c = nw + 32 * j + l32, h = c >> 7, d = c & 127;
      half* pr = ea.rk + ((size_t)h * ea.pp + mrow) * HDIM + d;
#pragma unroll
      for (int i = 0; i < FM; ++i) if (i >= ib && i < ie)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int rl = 32 * i + 8 * (v >> 2) + (v & 3);
          if (row_ok(rl)) pr[rl * HDIM] = to_f16(acc[i][j][v]);
        }
    }
  } else if constexpr (EPI == (int)Epi::StoreF16 || EPI == (int)Epi::StoreBF16 || EPI == (int)Epi::Silu ||
                       EPI == (int)Epi::BiasReluF16) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int c = nw + 32 * j + l32;
      const float bc = ea.bias ? ea.bias[c] : 0.0f;
      const size_t base = (size_t)mrow * ea.ldo + c;
#pragma unroll
      for (int i = 0; i < FM; ++i) if (i >= ib && i < ie)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int rl = 32 * i + 8 * (v >> 2) + (v & 3);
          if (!row_ok(rl)) continue;
          const size_t at = base + (size_t)rl * ea.ldo;
          const float x = acc[i][j][v];
          if constexpr (EPI == (int)Epi::StoreF16) {
            ea.out_f16[at] = to_f16(x + bc);
          } else if constexpr (EPI == (int)Epi::StoreBF16) {
            uint32_t u = __float_as_uint(x + bc);
            u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even (finite inputs)
            reinterpret_cast<uint16_t*>(ea.out_f16)[at] = (uint16_t)(u >> 16);
          } else if constexpr (EPI == (int)Epi::Silu) {
            ea.out_f16[at] = to_f16(fast_sigmoid_mul(x, x));
          } else {
            const float y = x + bc;
            ea.out_f16[at] = to_f16(y > 0.0f ? y : 0.0f);
          }
        }
    }
  } else {
#pragma unroll
    for (int i = 0; i < FM; ++i) if (i >= ib && i < ie)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = m0 + i * 32 + 8 * (v >> 2) + 4 * lhi + (v & 3);
          if (r < p.M) store_one<EPI>(ea, r, nw + 32 * j + l32, acc[i][j][v]);
        }
  }
  };
  // a tile inside M skips every per-row check (the f32 store, the split-K
  // partial, measured faster with the checks kept: one code path)
  if constexpr (EPI == (int)Epi::StoreF32 || EPI == (int)Epi::FlattenReluF16) epilogue(std::integral_constant<bool, true>());
  else if (m0 + 32 * FM <= p.M) epilogue(std::integral_constant<bool, false>());
  else epilogue(std::integral_constant<bool, true>());
}

// Wide-tile kernel: workgroup tile (32*FM) x 32*NB*WV, the WV waves (4; 1
// for short inputs, where 4-wave tiles would leave most CUs idle; 8 with one
// column block each, NB = 1, for launches of one round of tiles) side by
// side, each owning all rows and 32*NB columns (FM x NB MFMA blocks). Every output
// element is one MFMA chain over its k in the same order whatever FM and WV
// are, so the tile shape never changes results. B never
// touches LDS: an MFMA B fragment is 8 consecutive k of one weight row, i.e.
// one u32 of 4-bit codes (expanded in registers with the lane's two row
// tables) or 16 bytes of f16 weights. Only A is staged through LDS. The k
// order inside each 64-k tile is permuted identically on both operands (lane
// half h, slice s covers k = 32h + 8s .. +7), so a lane's B data for a whole
// k-tile is contiguous: one 16-byte load of codes or four of f16. Both weight
// formats therefore accumulate in the same order and give bit-identical
// results for the same weight values. Per k-tile a wave runs 8*FM MFMAs
// against 4*FM fragment reads (and 8 code expansions in 4-bit mode).
// K2ORD: accumulate slices 0-1 and 2-3 of every k-tile in two chains and add
// them at the end, the two-group kernel's order (used for its epilogues, so
// the tile shape still never changes results).
template <int FM, bool LUT4, bool SWZ, bool ABF16, int EPI, int WV = 4, bool K2ORD = false, int NB = 2>
__global__ void __launch_bounds__(64 * WV, (LUT4 && FM <= 4 && NB == 2) ? 2 : 1) gemm_wide_kernel(GemmParams p) {
  constexpr int NT = 64 * WV;  // threads: WV waves of 32 * NB columns each
  // plain 4-bit codes with bf16 activations (the isolated linear): A chunks
  // converted in the order the swizzled expansion gives plain codes
  constexpr bool EO = LUT4 && !SWZ && ABF16;
  constexpr int BM = 32 * FM;
  constexpr int A_CH = BM * BK / 8 / NT;  // 16-byte chunks of A per thread per k-tile
  constexpr int B_V = LUT4 ? NB : 4 * NB;  // 16-byte loads of B per lane per k-tile
  // 4-bit tiles of up to 128 rows keep two workgroups per CU (two waves per
  // SIMD, so one wave's code expansion overlaps the other's MFMAs): that needs
  // <= 256 registers per lane, hence two register stages of A and B.
  constexpr bool OCC2 = LUT4 && FM <= 4 && NB == 2;
  constexpr int BD = (LUT4 && !OCC2) ? 4 : 2;  // k-tiles of B in flight (register stages)
  constexpr int AD = (FM >= 6 || OCC2) ? 2 : 4;  // k-tiles of A in flight (register stages)
  __shared__ __attribute__((aligned(16))) half As[2][BM * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int l32 = lane & 31, lhi = lane >> 5;
  // XCD-aware tile order: the hardware hands block b to XCD b % 8, so block
  // ids are renumbered to give each XCD a contiguous run of tiles in (split,
  // row tile, column tile) order. All column tiles of a row tile then share
  // one XCD's L2 for their A rows (read once per row tile instead of once per
  // column tile). Which tile a workgroup computes does not change its results.
  const int gx = gridDim.x, gy = gridDim.y;
  const int G = gx * gy * gridDim.z;
  const int bid = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const int xq = G / 8, xr = G % 8, xcd = bid % 8;
  const int tix = xcd * xq + min(xcd, xr) + bid / 8;
  const int bz = tix / (gx * gy), by = (tix / gx) % gy, bx = tix % gx;
  const int n0 = bx * (32 * NB * WV), m0 = by * BM;
  const int nw = n0 + wid * 32 * NB;
  // K chunk of this split: whole 256-k units, the first K/256 % splits
  // chunks one unit longer (depends on K and the split count only)
  const int kunits = p.K / 256, kq = kunits / p.splits, kr = kunits % p.splits;
  const int kz0 = 256 * (bz * kq + min(bz, kr));  // first k of this split
  const int kc = 256 * (kq + (bz < kr ? 1 : 0));   // k of this split

  // Global addresses are a wave-uniform base plus 32-bit lane offsets (the
  // host checks the operands fit), so loads use scalar base registers.
  RowLut lut[NB];
  const uint8_t* bbase = LUT4 ? p.codes + kz0 / 2 : reinterpret_cast<const uint8_t*>(p.W + kz0);
  constexpr int B_ROW_BYTES_PER_K2 = LUT4 ? 1 : 4;  // bytes per row per 2 k
  uint32_t boff[NB];  // this lane's B bytes of k-tile 0, for its rows
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int n = nw + 32 * j + l32;
    // the register-held select mask except where it spills (two workgroups
    // per CU at 128 rows with the f32 partial-sum store)
    if constexpr (LUT4) lut[j] = load_row_lut<!(OCC2 && FM >= 4 && EPI == (int)Epi::StoreF32)>(p.lut + (size_t)n * 16);
    boff[j] = (uint32_t)n * (uint32_t)(p.K / 2 * B_ROW_BYTES_PER_K2) + (LUT4 ? 16 : 64) * lhi;
  }
  constexpr int B_TILE_BYTES = LUT4 ? BK / 2 : BK * 2;
  const half* abase = p.A + (size_t)m0 * p.lda + kz0;
  uint32_t aoff[A_CH];
  int a_lds[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int ch = tid + NT * i, row = ch >> 3, col = (ch & 7) * 8;
    aoff[i] = (uint32_t)min(row, p.M - 1 - m0) * (uint32_t)p.lda + col;  // rows past M repeat row M-1
    a_lds[i] = row * LDK + col;
  }

  struct AStage {
    uint4 v[A_CH];
  };
  struct BStage {
    uint4 v[B_V];
  };
  AStage ra0, ra1, ra2, ra3;
  BStage rb0, rb1, rb2, rb3;  // rb2/rb3 only with four B stages

  // Loads past the last k-tile re-read it (no branch, stays in bounds).
  const int nk = kc / BK;
  auto load_a_chunk = [&](int kt, AStage& a, int i) {
    kt = min(kt, nk - 1);
    a.v[i] = *reinterpret_cast<const uint4*>(abase + kt * BK + aoff[i]);
  };
  auto load_a = [&](int kt, AStage& a) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) load_a_chunk(kt, a, i);
  };
  auto load_b = [&](int kt, BStage& b) {
    kt = min(kt, nk - 1);
    const uint8_t* bt = bbase + (size_t)kt * B_TILE_BYTES;
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int q = 0; q < B_V / NB; ++q) b.v[j * (B_V / NB) + q] = *reinterpret_cast<const uint4*>(bt + boff[j] + 16 * q);
  };
  auto store_chunk = [&](int buf, const AStage& a, int i) {
    if constexpr (EO) {
      st_half8(&As[buf][a_lds[i]], bf16x8_to_f16_eo(uint4{a.v[i].x, a.v[i].y, a.v[i].z, a.v[i].w}));
    } else if constexpr (ABF16) {
      const uint32_t w4[4] = {a.v[i].x, a.v[i].y, a.v[i].z, a.v[i].w};
      half8 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = (half)__uint_as_float(w4[e] << 16);
        v[2 * e + 1] = (half)__uint_as_float(w4[e] & 0xffff0000u);
      }
      st_half8(&As[buf][a_lds[i]], v);
    } else {
      const uint4 t{a.v[i].x, a.v[i].y, a.v[i].z, a.v[i].w};
      *reinterpret_cast<uint4*>(&As[buf][a_lds[i]]) = t;
    }
  };

  floatx16 acc[FM][NB], acc_hi[K2ORD ? FM : 1][NB];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
  if constexpr (K2ORD)
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc_hi[i][j][v] = 0.0f;

  // A fragment row offset of block i for this lane, k slice s: chunk 4*lhi + s.
  const int af_off = l32 * LDK + 32 * lhi;
  auto read_af = [&](half8 (&af)[FM], int buf, int s) {
#pragma unroll
    for (int i = 0; i < FM; ++i) af[i] = ld_half8(&As[buf][af_off + i * 32 * LDK + 8 * s]);
  };
  auto code_word = [](const uint4& c, int s) { return s == 0 ? c.x : s == 1 ? c.y : s == 2 ? c.z : c.w; };
  auto b_frag = [&](const BStage& b, int j, int s) {
    uint4 q;
    if constexpr (LUT4) {
      q = expand8<SWZ || EO>(code_word(b.v[j], s), lut[j]);
    } else {
      q = uint4{b.v[4 * j + s].x, b.v[4 * j + s].y, b.v[4 * j + s].z, b.v[4 * j + s].w};
    }
    return *reinterpret_cast<const half8*>(&q);
  };

  // One k-tile from LDS buffer `cur` and B stage `bs`; meanwhile stores the
  // next tile's A (register stage `as`) into buffer `nxt`, and issues the
  // global loads of A k-tile `ka` into stage `ad` (slices 0-1) and of B k-tile
  // `kb` into stage `bd` (slice 3, after the last code word of `bs` was
  // expanded), spread between the MFMAs so the wave never stalls on a full
  // load queue with the matrix core idle.
  auto tile = [&](int cur, int nxt, const BStage& bs, const AStage& as, int ka, AStage& ad, int kb, BStage& bd) {
    half8 af[2][FM];
    half8 bf[2][NB];
    constexpr int VEXP = LUT4 ? 25 * NB : 1;  // VALU instructions of the slice's code expansions
    constexpr int VPER = (VEXP + NB * FM - 1) / (NB * FM);
    read_af(af[0], cur, 0);
#pragma unroll
    for (int j = 0; j < NB; ++j) bf[0][j] = b_frag(bs, j, 0);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int c = s & 1, n = c ^ 1;
      // slice s+1's fragment reads are issued before slice s's MFMAs (the
      // scheduler would otherwise sink them next to their use); the MFMAs
      // interleave with slice s+1's code expansions
      if (s < 3) read_af(af[n], cur, s + 1);
      __builtin_amdgcn_sched_barrier(0);
      if (s < 3) {
#pragma unroll
        for (int j = 0; j < NB; ++j) bf[n][j] = b_frag(bs, j, s + 1);
      }
#pragma unroll
      for (int i = 0; i < A_CH; ++i)
        if (i * 4 / A_CH == s) store_chunk(nxt, as, i);
      constexpr int A_LO = (A_CH + 1) / 2;
      if (s == 0) {
#pragma unroll
        for (int i = 0; i < A_LO; ++i) load_a_chunk(ka, ad, i);
      } else if (s == 1) {
#pragma unroll
        for (int i = A_LO; i < A_CH; ++i) load_a_chunk(ka, ad, i);
      } else if (s == 3) {
        load_b(kb, bd);
      }
      const int nvm = s == 0 ? A_LO : s == 1 ? A_CH - A_LO : s == 3 ? B_V : 0;  // loads this slice
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          if (K2ORD && s >= 2)
            acc_hi[K2ORD ? i : 0][j] =
                __builtin_amdgcn_mfma_f32_32x32x16_f16(af[c][i], bf[c][j], acc_hi[K2ORD ? i : 0][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[c][i], bf[c][j], acc[i][j], 0, 0, 0);
        }
#pragma unroll
      for (int m = 0; m < NB * FM; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (s < 3) __builtin_amdgcn_sched_group_barrier(0x002, VPER, 0);
        if (m < nvm) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Per k-tile kt: LDS buffer kt%2 holds A(kt); A(kt+1) is stored from its
  // register stage during the tile; loads for A(kt+AD) and B(kt+BD), issued
  // during the tile, refill the stages it frees. Past the end the stores repeat the last tile into
  // a buffer that is never read again.
  load_a(0, ra0);
  load_b(0, rb0);
  load_a(1, ra1);
  load_b(1, rb1);
  if constexpr (AD == 4) load_a(2, ra2);
  if constexpr (BD == 4) load_b(2, rb2);
  if constexpr (AD == 4) load_a(3, ra3);
  if constexpr (BD == 4) load_b(3, rb3);
#pragma unroll
  for (int i = 0; i < A_CH; ++i) store_chunk(0, ra0, i);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 4) {
    tile(0, 1, rb0, ra1, kt + AD, ra0, kt + BD, rb0);
    __syncthreads();
    tile(1, 0, rb1, AD == 4 ? ra2 : ra0, kt + 1 + AD, ra1, kt + 1 + BD, rb1);
    __syncthreads();
    tile(0, 1, BD == 4 ? rb2 : rb0, AD == 4 ? ra3 : ra1, kt + 2 + AD, AD == 4 ? ra2 : ra0, kt + 2 + BD,
         BD == 4 ? rb2 : rb0);
    __syncthreads();
    tile(1, 0, BD == 4 ? rb3 : rb1, ra0, kt + 3 + AD, AD == 4 ? ra3 : ra1, kt + 3 + BD, BD == 4 ? rb3 : rb1);
    __syncthreads();
  }
  if constexpr (K2ORD)
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] += acc_hi[i][j][v];

  tile_epilogue<FM, EPI, NB>(acc, p, m0, nw, bz, lane);
}

// Column-strip kernel for short inputs: a workgroup holds MW waves, one per
// 32-row block of a (32*MW)-row tile (blockIdx.y), and covers 32*NB columns
// (blockIdx.x) of one K chunk (blockIdx.z, chunked as in gemm_wide_kernel).
// Each k-tile's weight fragments (4 slices x NB column blocks, 1 KB each) are
// made ONCE per workgroup — fragment f by wave f % MW: expanded from the
// 4-bit codes with the row tables, or copied for f16 weights — into LDS, where
// every wave reads them; the A tile is staged through LDS from coalesced row
// loads (A fragments loaded straight from global memory touch 32 partial
// cache lines per instruction and measured 40 % slower). The one-wave wide tiles expand
// every code word once per 32 rows instead. Per-element order is the wide
// kernel's (k-tiles ascending, slices 0..3, lane half h of slice s covering
// k = 32h + 8s .. +7; K2ORD: slices 0-1 and 2-3 in two chains added at the
// end), so results are bit-identical to it. One barrier per k-tile: tile
// kt + 1's fragments go to the other LDS buffer while tile kt's are read.
template <bool LUT4, int EPI, int NB, bool K2ORD>
__global__ void __launch_bounds__(512) gemm_strip_kernel(GemmParams p) {
  constexpr int NF = 4 * NB;   // weight fragments per k-tile
  constexpr int FPW = 2 * NB;  // fragments one wave makes at most (MW >= 2)
  constexpr int SD = 4;        // k-tiles of A and weights in flight (register stages)
  __shared__ __attribute__((aligned(16))) uint4 Bs[2][NF][64];
  __shared__ __attribute__((aligned(16))) half As[2][256 * LDK];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int MW = blockDim.x >> 6;
  const int l32 = lane & 31, lhi = lane >> 5;
  const int n0 = blockIdx.x * 32 * NB, bz = blockIdx.z;
  const int m0 = (blockIdx.y * MW + wid) * 32;
  const int kunits = p.K / 256, kq = kunits / p.splits, kr = kunits % p.splits;
  const int kz0 = 256 * (bz * kq + min(bz, kr));
  const int nk = 4 * (kq + (bz < kr ? 1 : 0));  // k-tiles of this chunk

  // A staging: thread t loads 16-byte chunk t % 8 of rows t / 8 + 8 MW i
  // (i < 4) of the workgroup's rows (rows past M repeat row M - 1)
  const int wrow0 = blockIdx.y * MW * 32, arow = threadIdx.x >> 3, acol = (threadIdx.x & 7) * 8;
  const half* abase[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    abase[i] = p.A + (size_t)min(wrow0 + arow + 8 * MW * i, p.M - 1) * p.lda + kz0 + acol;
  const int af_off = (32 * wid + l32) * LDK + 32 * lhi;  // this lane's A fragments
  // weight data of the fragments this wave makes: fragment f = wid + MW * i
  // is column block j = f / 4, slice s = f % 4 of every k-tile
  // (the slice depends on the wave, a runtime value, so the load addresses its
  // code word directly: one 4-byte load, no runtime pick of a vector element)
  RowLut lut[FPW];
  const uint8_t* wsrc[FPW];
#pragma unroll
  for (int i = 0; i < FPW; ++i) {
    const int f = min(wid + MW * i, NF - 1), j = f >> 2, n = n0 + 32 * j + l32;
    if constexpr (LUT4) {
      lut[i] = load_row_lut(p.lut + (size_t)n * 16);
      wsrc[i] = p.codes + (size_t)n * (p.K / 2) + kz0 / 2 + 16 * lhi + 4 * (f & 3);  // 32 bytes per k-tile
    } else {
      wsrc[i] = reinterpret_cast<const uint8_t*>(p.W + (size_t)n * p.K + kz0 + 32 * lhi) + 16 * (f & 3);
    }
  }
  const int nmine = (NF - wid + MW - 1) / MW;  // fragments this wave makes

  // register stages: named variables, rotated by an unconditional four-tile
  // loop body (K chunks are whole 256-k units); their values reach LDS through
  // element-wise copies (a whole-member store through a cast pointer kept
  // every stage in scratch memory)
  using BW = std::conditional_t<LUT4, uint32_t, uint4>;  // one code word, or 8 f16 weights
  struct Stage {
    uint4 a[4];
    BW b[FPW];
  };
  Stage r0, r1, r2, r3;
  auto load = [&](int kt, Stage& st) __attribute__((always_inline)) {
    kt = min(kt, nk - 1);  // loads past the last k-tile re-read it
#pragma unroll
    for (int i = 0; i < 4; ++i) st.a[i] = *reinterpret_cast<const uint4*>(abase[i] + kt * BK);
#pragma unroll
    for (int i = 0; i < FPW; ++i)
      if (i < nmine) st.b[i] = *reinterpret_cast<const BW*>(wsrc[i] + kt * (LUT4 ? BK / 2 : BK * 2));
  };
  auto make = [&](int buf, const Stage& st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FPW; ++i) {
      if (i < nmine) {
        if constexpr (LUT4) {
          Bs[buf][wid + MW * i][lane] = expand8<true>(st.b[i], lut[i]);
        } else {
          const uint4 t{st.b[i].x, st.b[i].y, st.b[i].z, st.b[i].w};
          Bs[buf][wid + MW * i][lane] = t;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 t{st.a[i].x, st.a[i].y, st.a[i].z, st.a[i].w};
      *reinterpret_cast<uint4*>(&As[buf][(arow + 8 * MW * i) * LDK + acol]) = t;
    }
  };

  floatx16 acc[1][NB], acc_hi[K2ORD ? NB : 1];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[0][j][v] = 0.0f;
  if constexpr (K2ORD)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc_hi[j][v] = 0.0f;

  auto mfmas = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const half8 af = ld_half8(&As[buf][af_off + 8 * s]);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const uint4 b4 = Bs[buf][4 * j + s][lane];
        const half8 bf = *reinterpret_cast<const half8*>(&b4);
        if (K2ORD && s >= 2)
          acc_hi[K2ORD ? j : 0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc_hi[K2ORD ? j : 0], 0, 0, 0);
        else
          acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[0][j], 0, 0, 0);
      }
    }
  };

  // k-tile kt lives in register stage kt % 4 and LDS buffer kt % 2; past the
  // last tile, loads re-read it and the fragments made go to a buffer that is
  // never read again
  // the tile's MFMAs are issued first and the next tile's fragments (the
  // other LDS buffer) are made between them
  auto iter = [&](int kt, Stage& cur, const Stage& next) __attribute__((always_inline)) {
    load(kt + SD, cur);  // stage kt % 4's tile kt is already in LDS
    mfmas(kt & 1);
    make((kt + 1) & 1, next);
#pragma unroll
    for (int m = 0; m < 4 * NB; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);             // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, LUT4 ? 8 : 1, 0);  // a few VALU
    }
    __syncthreads();
  };
  load(0, r0);
  load(1, r1);
  load(2, r2);
  load(3, r3);
  make(0, r0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += SD) {
    iter(kt, r0, r1);
    iter(kt + 1, r1, r2);
    iter(kt + 2, r2, r3);
    iter(kt + 3, r3, r0);
  }
  if constexpr (K2ORD)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[0][j][v] += acc_hi[j][v];
  if (m0 >= p.M) return;  // a wave past the last row (no barrier follows)
  tile_epilogue<1, EPI, NB>(acc, p, m0, n0, bz, lane);
}

// Two-group tile kernel: 512 threads = two K-groups of four waves. Wave
// (g, w) computes the same (32*FM) x 64 tile as wave w of gemm_wide_kernel;
// of every 64-k tile, group g runs the 16-k slices 2g and 2g + 1 (k = 32h +
// 8s .. +7 for lane half h, slice s, the wide kernel's permuted order). Waves
// w and w + 4 share a SIMD, so every SIMD runs two waves of one tile and one
// wave's code expansion (VALU) proceeds while the other's MFMAs do: within
// one wave the two barely overlap, across two waves of a SIMD they do
// (measured on MI355X). Launches with fewer tiles than CUs therefore still
// run two waves per SIMD.
//
// Operands reach LDS by direct global->LDS loads (global_load_lds_dwordx4, 16
// bytes per lane, no staging registers), issued NS - 1 k-tiles ahead into NS
// stages shared by both groups:
//  - A in unpadded 128-byte rows whose 16-byte chunks are XOR-swizzled by row
//    pair (chunk c of row r at position c ^ ((r >> 1) & 7)): LDS serves 256
//    bytes per clock, two 128-byte rows side by side, so the fragment reads of
//    16 consecutive lanes (rows r .. r + 15) hit 16 distinct bank groups;
//  - 4-bit weights: the 32 code bytes of each of the tile's 256 rows, read
//    back by the lanes that expand them (row tables stay in registers);
//    f16 weights: 128-byte rows swizzled like A.
// The loads are issued from inline asm, so the compiler does not track them:
// each wave waits for its own loads of a stage (vmcnt) and a workgroup
// barrier follows before any use; nothing else in the loop reads global
// memory. bf16 activations are converted to f16 in place after they land.
// Both weight formats run the same MFMA sequence, so equal weight values give
// bit-identical results. At the end group 1 hands its accumulators to group 0
// through LDS; group 0 adds them (a fixed order) and runs the epilogue.
template <int FM, bool LUT4>
struct K2Shape {
  // LDS stages (loads run NS - 1 k-tiles ahead); 4-bit tiles are small
  // enough for four
  static constexpr int NS = LUT4 ? 4 : 3;
  static constexpr int A_BYTES = 32 * FM * BK * 2;                  // A of one k-tile
  static constexpr int B_BYTES = LUT4 ? 256 * BK / 2 : 256 * BK * 2;  // weights of one k-tile
  static constexpr int ST_BYTES = A_BYTES + B_BYTES;
  static constexpr int A_INSTR = A_BYTES / 1024;                    // wave-level loads of A (= 4 FM)
  static constexpr int B_INSTR = B_BYTES / 1024;                    // and of the weights (8 or 32)
  static constexpr int A_HI = (A_INSTR + 7) / 8, A_LO = A_INSTR / 8;  // per wave (waves < A_INSTR % 8: A_HI)
  static constexpr int B_PER = B_INSTR / 8;
  static constexpr int HALF = (FM + 1) / 2;                         // row blocks exchanged per round
  static constexpr size_t STAGES = (size_t)NS * ST_BYTES;
  static constexpr size_t XCHG = (size_t)HALF * 4 * 2 * 16 * 64 * 4;
  static constexpr size_t STAGING = (size_t)2 * 32 * 260 * 4;      // epilogue tiles of both groups
  static constexpr size_t LDS0 = STAGES > XCHG ? STAGES : XCHG;
  static constexpr size_t LDS = LDS0 > STAGING ? LDS0 : STAGING;
};

// global -> LDS, 16 bytes per lane: lane l's bytes at gbase + voff land at
// LDS byte address lds + 16 l (gbase and lds wave-uniform). M0 carries the LDS
// address; nothing else in the kernels using this relies on M0.
__device__ inline void dma16(const void* gbase, uint32_t voff, uint32_t lds) {
  // the base and the LDS address are wave-uniform by contract; readfirstlane
  // puts them in scalar registers whatever the divergence analysis concluded
  // (readfirstlane returns int: each half goes through uint32_t before it is
  // widened, or a low half with bit 31 set would sign-extend into the high one)
  const uint64_t g = (uint64_t)(uintptr_t)gbase;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(g >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)g);
  const uint64_t gs = ((uint64_t)hi << 32) | (uint64_t)lo;
  const uint32_t ls = (uint32_t)__builtin_amdgcn_readfirstlane(lds);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(gs), "s"(ls) : "memory", "m0");
#pragma clang diagnostic pop
}

// s_waitcnt with only vmcnt constrained (expcnt, lgkmcnt at their maxima)
template <int N>
__device__ inline void wait_vmcnt_le() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// Epilogue of the two-group kernel. Each group finishes its row blocks one
// 32-row block per round: the block's f32 sums go to the group's LDS staging
// tile (32 x 256, rows padded to K2_XLD floats), then the group's 256 threads
// apply the epilogue arithmetic of tile_epilogue / store_one element by
// element and store 16-byte runs along the output's contiguous dimension: 8
// columns of a row (row-major outputs, head-major q / k / relK rows), 8 rows of
// a column (the transposed V), 4 GLU channels of a row (f32).
constexpr int K2_XLD = 260;

__device__ inline uint16_t bf16_bits(float v) {
  uint32_t u = __float_as_uint(v);
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even (finite inputs)
  return (uint16_t)(u >> 16);
}

// Stores staged block rows [0, 32) (global rows row0 ..) x tile columns [0, 256).
template <int EPI>
__device__ inline void k2_store_block(const float* xs, const GemmParams& p, int row0, int n0, int bz, int gt) {
  const EpiArgs& ea = p.ea;
  if constexpr (EPI == (int)Epi::Glu) {
    // output channel (n0 >> 1) + ch: value = column 64 (ch >> 5) + (ch & 31), gate = that + 32
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int q = gt + 256 * k, row = q >> 5, ch = (q & 31) * 4;
      if (row0 + row >= p.M) continue;
      const int cv = 64 * (ch >> 5) + (ch & 31);
      const floatx4 a = *reinterpret_cast<const floatx4*>(xs + row * K2_XLD + cv);
      const floatx4 g = *reinterpret_cast<const floatx4*>(xs + row * K2_XLD + cv + 32);
      floatx4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = fast_sigmoid_mul(a[e], g[e]);
      *reinterpret_cast<floatx4*>(ea.out_f32 + (size_t)(row0 + row) * ea.ldo + (n0 >> 1) + ch) = o;
    }
  } else if constexpr (EPI == (int)Epi::Qkv) {
    const int region = n0 >> 10;  // 0 q, 1 k, 2 v (a tile lies in one)
    if (region == 2) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int q = gt + 256 * k, c = q >> 2, r8 = (q & 3) * 8;
        const int hd = n0 - 2048 + c;
        half* dst = ea.vt + (size_t)hd * ea.mp + row0 + r8;
        half8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = to_f16(xs[(r8 + e) * K2_XLD + c]);
        if (row0 + r8 + 7 < p.M) {
          *reinterpret_cast<half8*>(dst) = o;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (row0 + r8 + e < p.M) dst[e] = o[e];
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int q = gt + 256 * k, row = q >> 5, c8 = (q & 31) * 8;
        if (row0 + row >= p.M) continue;
        const int hd = (n0 & 1023) + c8, h = hd >> 7, d = hd & 127;
        const size_t off = ((size_t)h * ea.mp + row0 + row) * HDIM + d;
        const floatx4 a = *reinterpret_cast<const floatx4*>(xs + row * K2_XLD + c8);
        const floatx4 b = *reinterpret_cast<const floatx4*>(xs + row * K2_XLD + c8 + 4);
        const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        if (region == 0) {
          half8 u, w;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            u[e] = to_f16((v[e] + ea.bu[hd + e]) * ea.scale);
            w[e] = to_f16((v[e] + ea.bv[hd + e]) * ea.scale);
          }
          *reinterpret_cast<half8*>(ea.qu + off) = u;
          *reinterpret_cast<half8*>(ea.qv + off) = w;
        } else {
          half8 u;
#pragma unroll
          for (int e = 0; e < 8; ++e) u[e] = to_f16(v[e]);
          *reinterpret_cast<half8*>(ea.kh + off) = u;
        }
      }
    }
  } else {
    // row-major outputs and relK (head-major rows): 8 columns of a row
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int q = gt + 256 * k, row = q >> 5, c8 = (q & 31) * 8;
      if (row0 + row >= p.M) continue;
      const int grow = row0 + row, col = n0 + c8;
      const floatx4 a = *reinterpret_cast<const floatx4*>(xs + row * K2_XLD + c8);
      const floatx4 b = *reinterpret_cast<const floatx4*>(xs + row * K2_XLD + c8 + 4);
      float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
      if constexpr (EPI == (int)Epi::StoreF32) {
        float* dst = ea.out_f32 + bz * p.out_zstride + (size_t)grow * ea.ldo + col;
        if (ea.bias) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] += ea.bias[col + e];
        }
        *reinterpret_cast<floatx4*>(dst) = floatx4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<floatx4*>(dst + 4) = floatx4{v[4], v[5], v[6], v[7]};
      } else if constexpr (EPI == (int)Epi::StoreF16 || EPI == (int)Epi::Silu) {
        half8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (EPI == (int)Epi::Silu) o[e] = to_f16(fast_sigmoid_mul(v[e], v[e]));
          else o[e] = to_f16(ea.bias ? v[e] + ea.bias[col + e] : v[e]);
        }
        *reinterpret_cast<half8*>(ea.out_f16 + (size_t)grow * ea.ldo + col) = o;
      } else if constexpr (EPI == (int)Epi::StoreBF16) {
        uint16_t o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = bf16_bits(ea.bias ? v[e] + ea.bias[col + e] : v[e]);
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(ea.out_f16) + (size_t)grow * ea.ldo + col) =
            *reinterpret_cast<const uint4*>(o);
      } else if constexpr (EPI == (int)Epi::RelK) {
        const int h = col >> 7, d = col & 127;
        half8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = to_f16(v[e]);
        *reinterpret_cast<half8*>(ea.rk + ((size_t)h * ea.pp + grow) * HDIM + d) = o;
      }
    }
  }
}

template <int FM, bool LUT4, bool SWZ, bool ABF16, int EPI>
__global__ void __launch_bounds__(512, 1) gemm_k2_kernel(GemmParams p) {
  using S = K2Shape<FM, LUT4>;
  constexpr int NS = S::NS;
  extern __shared__ __attribute__((aligned(16))) unsigned char k2_lds[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave 0..7
  const int grp = wv >> 2, w = wv & 3;
  const int l32 = lane & 31, lhi = lane >> 5;
  // XCD-aware tile order, as gemm_wide_kernel
  const int gx = gridDim.x, gy = gridDim.y;
  const int G = gx * gy * gridDim.z;
  const int bid = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const int xq = G / 8, xr = G % 8, xcd = bid % 8;
  const int tix = xcd * xq + min(xcd, xr) + bid / 8;
  const int bz = tix / (gx * gy), by = (tix / gx) % gy, bx = tix % gx;
  const int n0 = bx * 256, m0 = by * 32 * FM;
  const int nw = n0 + w * 64;
  const int kunits = p.K / 256, kq = kunits / p.splits, kr = kunits % p.splits;
  const int kz0 = 256 * (bz * kq + min(bz, kr));
  const int nk = 4 * (kq + (bz < kr ? 1 : 0));  // k-tiles of this split

  // this lane's row tables, complete before any load is issued (the compiler
  // only knows of these loads)
  RowLut lut[2];
  if constexpr (LUT4) {
#pragma unroll
    for (int j = 0; j < 2; ++j)  // the register form where it does not spill (SiLU)
      lut[j] = load_row_lut<EPI == (int)Epi::Silu>(p.lut + (size_t)(nw + 32 * j + l32) * 16);
  }
  wait_vmcnt_le<0>();

  // Load sources. Wave-level load d of a k-tile writes LDS bytes 1024 d ..
  // of the stage, chunk ch = 64 d + lane: A row ch >> 3 at position ch & 7,
  // holding global chunk (ch & 7) ^ ((row >> 1) & 7) (rows past M repeat row M - 1,
  // never stored). Wave wv issues A loads d = wv, wv + 8, ... and weight loads
  // d = wv + 8 t (t < B_PER): 4-bit, chunk P = 64 d + lane is row P >> 1, code
  // bytes 16 (P & 1) .. of the row's 32; f16, row ch >> 3 like A.
  const int a_my = wv < S::A_INSTR % 8 ? S::A_HI : S::A_LO;
  const half* abase = p.A + (size_t)m0 * p.lda + kz0;
  uint32_t aoff[S::A_HI];
#pragma unroll
  for (int t = 0; t < S::A_HI; ++t) {
    const int ch = 64 * (wv + 8 * t) + lane, row = min(ch >> 3, 32 * FM - 1), cc = (ch & 7) ^ ((row >> 1) & 7);
    aoff[t] = ((uint32_t)min(row, p.M - 1 - m0) * (uint32_t)p.lda + cc * 8) * 2u;
  }
  const uint8_t* bbase = LUT4 ? p.codes + (size_t)n0 * (p.K / 2) + kz0 / 2
                              : reinterpret_cast<const uint8_t*>(p.W + (size_t)n0 * p.K + kz0);
  uint32_t boff[S::B_PER];
#pragma unroll
  for (int t = 0; t < S::B_PER; ++t) {
    const int ch = 64 * (wv + 8 * t) + lane;
    if constexpr (LUT4) {
      boff[t] = (uint32_t)(ch >> 1) * (uint32_t)(p.K / 2) + 16 * (ch & 1);
    } else {
      const int row = ch >> 3, cc = (ch & 7) ^ ((row >> 1) & 7);
      boff[t] = ((uint32_t)row * (uint32_t)p.K + cc * 8) * 2u;
    }
  }
  const uint32_t lds0 = lds_addr(k2_lds);

  // k-tile kt into stage st (loads past the last k-tile re-read it: in
  // bounds, and their stage is never read)
  auto issue = [&](int kt, int st) {
    kt = min(kt, nk - 1);
    const uint32_t sb = lds0 + st * S::ST_BYTES;
    const half* at = abase + kt * BK;
#pragma unroll
    for (int t = 0; t < S::A_HI; ++t)
      if (t < a_my) dma16(at, aoff[t], sb + (wv + 8 * t) * 1024);
    const uint8_t* bt = bbase + (size_t)kt * (LUT4 ? BK / 2 : BK * 2);
#pragma unroll
    for (int t = 0; t < S::B_PER; ++t) dma16(bt, boff[t], sb + S::A_BYTES + (wv + 8 * t) * 1024);
  };
  // a wave waits for its own loads of the oldest stage in flight: those of
  // the NS - 2 k-tiles issued after them may stay outstanding
  auto wait_stage = [&]() {
    if (wv < S::A_INSTR % 8) wait_vmcnt_le<(NS - 2) * (S::A_HI + S::B_PER)>();
    else wait_vmcnt_le<(NS - 2) * (S::A_LO + S::B_PER)>();
  };
  // bf16 activations: each wave converts the A chunks it loaded, in place
  auto convert_a = [&](int st) {
    if constexpr (ABF16) {
      half* a = reinterpret_cast<half*>(k2_lds + st * S::ST_BYTES);
#pragma unroll
      for (int t = 0; t < S::A_HI; ++t) {
        if (t >= a_my) continue;
        half* c = a + (64 * (wv + 8 * t) + lane) * 8;
        const uint4 u = *reinterpret_cast<const uint4*>(c);
        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
        half8 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = (half)__uint_as_float(w4[e] << 16);
          v[2 * e + 1] = (half)__uint_as_float(w4[e] & 0xffff0000u);
        }
        st_half8(c, v);
      }
    }
  };

  floatx16 acc[FM][2];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int arow_sw = (l32 >> 1) & 7;
  // Fragments of this group's two slices of one k-tile: A (both slices) and
  // the weights, 4-bit codes expanded to f16 — read and expanded in one phase,
  // multiplied in the next.
  half8 af[2][FM], bf[2][2];
  auto load_frags = [&](int st) {
    const unsigned char* sb = k2_lds + st * S::ST_BYTES;
    const half* a = reinterpret_cast<const half*>(sb);
    const unsigned char* bw = sb + S::A_BYTES;
    uint2 cw[2];
    if constexpr (LUT4) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        cw[j] = *reinterpret_cast<const uint2*>(bw + ((w * 64 + 32 * j + l32) * 2 + lhi) * 16 + 8 * grp);
    }
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
      const int s = 2 * grp + ss;
      const half* ar = a + l32 * BK + (((4 * lhi + s) ^ arow_sw) * 8);
#pragma unroll
      for (int i = 0; i < FM; ++i) af[ss][i] = ld_half8(ar + i * 32 * BK);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if constexpr (LUT4) {
          const uint4 q = expand8<SWZ>(ss == 0 ? cw[j].x : cw[j].y, lut[j]);
          bf[ss][j] = *reinterpret_cast<const half8*>(&q);
        } else {
          const int col = w * 64 + 32 * j + l32;
          bf[ss][j] = ld_half8(reinterpret_cast<const half*>(bw) + col * BK + (((4 * lhi + s) ^ ((col >> 1) & 7)) * 8));
        }
      }
    }
  };
  auto mfma_all = [&]() {
#pragma unroll
    for (int ss = 0; ss < 2; ++ss)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[ss][i], bf[ss][j], acc[i][j], 0, 0, 0);
  };

  // Ping-pong: the two waves of a SIMD run opposite phases. In phase 1 of
  // k-tile t group 0 multiplies tile t (fragments prepared in the phase
  // before) while group 1 reads and expands tile t; in phase 2 group 1
  // multiplies tile t while group 0 prepares tile t + 1. So one wave's MFMAs
  // overlap the other's LDS reads and code expansion. During phase 1 every
  // wave issues its loads of tile t + 2 into the stage tile t - 1 occupied
  // (both groups finished with it by the barrier that ended the previous
  // k-tile), then waits for its own loads of tile t + 1; the barrier after
  // phase 1 makes tile t + 1 visible to all waves for the reads of phase 2.
  // (the group is a template constant in each copy of the loop, so the
  // compiler sees when the fragments are dead; both copies execute the same
  // barriers)
  auto pingpong = [&](auto gconst) {
    constexpr int G = decltype(gconst)::value;
#pragma unroll
    for (int t = 0; t < NS - 1; ++t) issue(t, t);
    __builtin_amdgcn_sched_barrier(0);
    wait_stage();
    __builtin_amdgcn_s_barrier();
    if constexpr (ABF16) {
      convert_a(0);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_s_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (G == 0) load_frags(0);
    for (int kt = 0; kt < nk; ++kt) {
      const int st = kt % NS;
      __builtin_amdgcn_sched_barrier(0);
      // phase 1
      if constexpr (G == 0) mfma_all();
      else load_frags(st);
      __builtin_amdgcn_sched_barrier(0);
      issue(kt + NS - 1, (kt + NS - 1) % NS);
      __builtin_amdgcn_sched_barrier(0);
      wait_stage();
      __builtin_amdgcn_s_barrier();
      if constexpr (ABF16) {
        if (kt + 1 < nk) convert_a((kt + 1) % NS);
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_s_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
      // phase 2
      if constexpr (G == 1) mfma_all();
      else if (kt + 1 < nk) load_frags((kt + 1) % NS);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
    }
  };
  if (grp == 0) pingpong(std::integral_constant<int, 0>());
  else pingpong(std::integral_constant<int, 1>());
  wait_vmcnt_le<0>();
  __syncthreads();  // every load landed and every wave is done with the stages

  // The two groups' sums are combined through LDS and both groups finish
  // the tile: group 0 the row blocks [0, H0), group 1 the rest. Round 0: group
  // 1 hands over its blocks [0, H0); round 1: group 0 its blocks [H0, FM).
  // (acc_g0 + acc_g1 either way: the addition commutes exactly.)
  float* xb = reinterpret_cast<float*>(k2_lds);
  constexpr int H0 = S::HALF;
  auto xaddr = [&](int bi, int j, int q) { return xb + (((((w * H0 + bi) * 2 + j) * 4 + q) * 64 + lane) * 4); };
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int i0 = r == 0 ? 0 : H0, i1 = r == 0 ? H0 : FM;
    if (grp == 1 - r) {  // sender
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if (i < i0 || i >= i1) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const floatx4 v4 = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            *reinterpret_cast<floatx4*>(xaddr(i - i0, j, q)) = v4;
          }
      }
    }
    __syncthreads();
    if (grp == r) {  // receiver
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if (i < i0 || i >= i1) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const floatx4 v4 = *reinterpret_cast<const floatx4*>(xaddr(i - i0, j, q));
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v4[e];
          }
      }
    }
    if (r == 0) __syncthreads();
  }
  // Per-element epilogue (both groups at once, each on its blocks), except
  // the transposed V of the qkv projection: its 16-byte runs go down a column,
  // so those tiles are staged through LDS one 32-row block per round.
  if constexpr (EPI == (int)Epi::Qkv) {
    if (n0 >= 2048) {
      __syncthreads();  // the exchange area is reused for staging
      float* xs = xb + grp * 32 * K2_XLD;
      const int gt = w * 64 + lane;
#pragma unroll
      for (int r = 0; r < H0; ++r) {
        const int bi = grp == 0 ? r : H0 + r;  // this group's block of the round
        const bool active = bi < FM;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          if (i != bi) continue;
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              xs[(8 * (v >> 2) + 4 * lhi + (v & 3)) * K2_XLD + 64 * w + 32 * j + l32] = acc[i][j][v];
        }
        __syncthreads();
        if (active) k2_store_block<EPI>(xs, p, m0 + 32 * bi, n0, bz, gt);
        __syncthreads();
      }
      return;
    }
  }
  if (grp == 0) tile_epilogue<FM, EPI>(acc, p, m0, nw, bz, lane, 0, H0);
  else tile_epilogue<FM, EPI>(acc, p, m0, nw, bz, lane, H0, FM);
}


// out[r][c] = sum_s part[s][r][c] (s ascending), stored as f32 / f16 / bf16
// (out_kind 0 / 1 / 2, bf16 rounded to nearest even). Four columns per thread.
__global__ void __launch_bounds__(256) split_reduce_kernel(const float* part, int splits, size_t stride,
                                                           void* out, int out_kind, long n4) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  floatx4 v = reinterpret_cast<const floatx4*>(part)[i];
  for (int s = 1; s < splits; ++s) {
    const floatx4 q = reinterpret_cast<const floatx4*>(part + s * stride)[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += q[e];
  }
  if (out_kind == 0) {
    reinterpret_cast<floatx4*>(out)[i] = v;
  } else if (out_kind == 1) {
    const half4 h = {(half)v[0], (half)v[1], (half)v[2], (half)v[3]};
    reinterpret_cast<half4*>(out)[i] = h;
  } else {
    uint16_t b[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t u = __float_as_uint(v[e]);
      u += 0x7fffu + ((u >> 16) & 1u);
      b[e] = (uint16_t)(u >> 16);
    }
    reinterpret_cast<uint2*>(out)[i] = make_uint2(b[0] | ((uint32_t)b[1] << 16), b[2] | ((uint32_t)b[3] << 16));
  }
}

// ---------------------------------------------------------------------------
// Skinny kernel: the isolated 4-bit linear at M <= 256 (short utterances),
// where streaming the weights is the whole cost. The output is computed
// transposed, C^T = W . A^T, so the weights are the MFMA's row operand: a
// lane's 16-byte code load is 32 consecutive k of one output column, expanded
// in registers into four 8-k fragments (MFMA k slots may hold any k, as long
// as both operands agree: step c of a 64-k chunk takes k + 8c .. + 7 in lane
// half 0 and k + 32 + 8c .. + 7 in lane half 1).
//
// A workgroup owns 32 output columns and 32 * MB rows; its four waves take
// one quarter of K each and are summed through LDS in wave order (a fixed
// order: results do not depend on timing). Each wave stages its activation
// chunk (32 * MB rows x 64 k) through its own LDS region: loaded row by row
// (eight rows of 128 bytes per load instruction, where fragment-shaped loads
// touch 32-64 cache lines each and ran at the vector L1's line rate),
// converted from bf16 on the way when needed (in the k order that lets the
// plain codes take the swizzled expansion, bf16x8_to_f16_eo), and read back as MFMA
// fragments. The next chunk's codes and activations are in flight meanwhile.
// Rows are split over workgroups, never K, so no partial sums leave the
// workgroup (a K split finished by the last-arriving workgroup needed an
// agent-scope release per workgroup, an L2 write-back that cost more than
// the split saved).
constexpr int SK_LD = 72;  // halves per staged activation row (64 used; 144 bytes)

struct SkinnyArgs {
  GemmParams p;
  void* out;
  int out_kind;  // 0 f32, 1 f16, 2 bf16
};

// rows m, columns n .. n + 3 of C from one lane's four accumulators
__device__ inline void skinny_store4(const SkinnyArgs& s, int m, int n, floatx4 v) {
  const size_t o = (size_t)m * s.p.N + n;
  if (s.out_kind == 0) {
    *reinterpret_cast<floatx4*>(static_cast<float*>(s.out) + o) = v;
  } else if (s.out_kind == 1) {
    const half4 h = {to_f16(v[0]), to_f16(v[1]), to_f16(v[2]), to_f16(v[3])};
    *reinterpret_cast<half4*>(static_cast<half*>(s.out) + o) = h;
  } else {
    uint32_t b[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t u = __float_as_uint(v[e]);
      u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even (finite inputs)
      b[e] = u >> 16;
    }
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(s.out) + o) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
  }
}

template <int MB, bool ABF16>
__global__ void __launch_bounds__(256, 2) gemm_skinny_kernel(SkinnyArgs s) {
  constexpr int ROWS = 32 * MB;
  constexpr int LD_PER = ROWS / 8;  // row loads per lane per chunk (eight rows of 128 B per wave load)
  __shared__ __attribute__((aligned(16))) half stage[4][ROWS * SK_LD];
  floatx4* red = reinterpret_cast<floatx4*>(&stage[0][0]);  // [wave][row block][quad][lane], after the loop
  static_assert(sizeof(stage) >= 4 * MB * 4 * 64 * sizeof(floatx4), "reduction fits the staging area");
  const GemmParams& p = s.p;
  const int n0 = blockIdx.x * 32, m0 = blockIdx.y * ROWS;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, lhi = lane >> 5;
  const int kq = p.K / 4, kw0 = w * kq;
  const int n = n0 + l32;
  const RowLut lut = load_row_lut(p.lut + (size_t)n * 16);
  const uint8_t* crow = p.codes + (size_t)n * (p.K / 2) + 16 * lhi;
  // staging loads: lane reads row (8 i + lane / 8), bytes 16 (lane % 8) .. + 15 of the chunk
  const int sr = lane >> 3, sc = (lane & 7) * 8;
  const half* abase[LD_PER];
#pragma unroll
  for (int i = 0; i < LD_PER; ++i)  // rows >= M read row M - 1 and are not stored
    abase[i] = p.A + (size_t)min(m0 + 8 * i + sr, p.M - 1) * p.lda + sc;
  int nld = 0;  // row loads that hit rows < M (uniform)
#pragma unroll
  for (int i = 0; i < LD_PER; ++i) nld += m0 + 8 * i < p.M;
  half* const st = stage[w];

  floatx16 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[mb][v] = 0.0f;
  uint4 cw = *reinterpret_cast<const uint4*>(crow + kw0 / 2);
  uint4 ar[LD_PER] = {};  // rows past the end stay zero
  auto load_a = [&](int kc) {
#pragma unroll
    for (int i = 0; i < LD_PER; ++i)
      if (i < nld) ar[i] = *reinterpret_cast<const uint4*>(abase[i] + kc);
  };
  auto wave_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  load_a(kw0);
  for (int kc = kw0; kc < kw0 + kq; kc += 64) {
    wave_sync();  // the previous chunk's fragment reads are done
#pragma unroll
    for (int i = 0; i < LD_PER; ++i) {
      const half8 v = ABF16 ? bf16x8_to_f16_eo(ar[i]) : __builtin_bit_cast(half8, ar[i]);
      st_half8(st + (8 * i + sr) * SK_LD + sc, v);
    }
    const uint32_t words[4] = {cw.x, cw.y, cw.z, cw.w};
    if (kc + 64 < kw0 + kq) {  // uniform: the next chunk in flight
      cw = *reinterpret_cast<const uint4*>(crow + (kc + 64) / 2);
      load_a(kc + 64);
    }
    half8 wf[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) wf[c] = __builtin_bit_cast(half8, expand8<ABF16>(words[c], lut));
    wave_sync();  // the staged rows are visible to the whole wave
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      if (m0 + 32 * mb < p.M)  // uniform: row blocks past the end
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const half8 af = ld_half8(st + (32 * mb + l32) * SK_LD + 32 * lhi + 8 * c);
          acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[c], af, acc[mb], 0, 0, 0);
        }
    }
  }

  // the four K quarters, summed in wave order; wave w finishes row block w
  __syncthreads();  // every wave is done with its staging area
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      red[((w * MB + mb) * 4 + g) * 64 + lane] =
          floatx4{acc[mb][4 * g], acc[mb][4 * g + 1], acc[mb][4 * g + 2], acc[mb][4 * g + 3]};
  __syncthreads();
  const int mb = w;
  const int m = m0 + 32 * mb + l32;
  if (mb >= MB || m >= p.M) return;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    floatx4 x = red[((0 * MB + mb) * 4 + g) * 64 + lane];
#pragma unroll
    for (int q = 1; q < 4; ++q) {
      const floatx4 y = red[((q * MB + mb) * 4 + g) * 64 + lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] += y[e];
    }
    skinny_store4(s, m, n0 + 8 * g + 4 * lhi, x);
  }
}

// Skinny-kernel rows per workgroup (MB row blocks of 32): one block, which
// gives the most workgroups (6 x N / 32 at T = 188) and measured fastest on
// MI355X for all three config-1 shapes (a sweep of 1-4 blocks: 9.3 / 13.7 /
// 8.7 us at MB = 1 against 9.8 / 23.6 / 9.3 at MB = 3, T = 188; each phase is
// latency-bound, so more resident workgroups win over less code expansion).
// BARK_HIP_SKINNY_MB = 1..4 forces a count. 0 when the kernel does not apply.
int skinny_mb(int M, int N, int K) {
  if (M < 1 || M > 256 || N % 32 != 0 || K % 256 != 0) return 0;
  static const int forced = [] {
    const char* e = getenv("BARK_HIP_SKINNY_MB");
    return e ? atoi(e) : 0;
  }();
  return forced >= 1 && forced <= 4 ? forced : 1;
}

template <int MB>
void launch_skinny_mb(const SkinnyArgs& a, bool abf16, hipStream_t st) {
  const dim3 grid(a.p.N / 32, ceil_div(a.p.M, 32 * MB)), block(256);
  if (abf16) BARK_LAUNCH((gemm_skinny_kernel<MB, true>), grid, block, 0, st, a);
  else BARK_LAUNCH((gemm_skinny_kernel<MB, false>), grid, block, 0, st, a);
}

// Weight format: 0 = f16, 1 = swizzled 4-bit (encoder), 2 = plain 4-bit
// (isolated linear; f16 or bf16 activations). Only the combinations the
// encoder and the isolated linear use are instantiated; wide_supported()
// tells the dispatcher which ones exist (the rest run on the 128-column
// kernel).
bool wide_supported(Epi epi, int fmt) {
  if (fmt == 2) return epi == Epi::StoreF32 || epi == Epi::StoreF16 || epi == Epi::StoreBF16;
  switch (epi) {
    case Epi::StoreF32:
    case Epi::Silu:
    case Epi::Glu:
    case Epi::Qkv:
    case Epi::RelK:
    case Epi::BiasReluF16:
    case Epi::FlattenReluF16:
      return true;
    default:
      return false;
  }
}

template <int FM, int WV = 4, bool K2ORD = false, int NB = 2>
void launch_wide(const GemmParams& p, Epi epi, int fmt, bool abf16, hipStream_t s) {
  BARK_REQUIRE(p.N % (32 * NB * WV) == 0, "gemm: N is not a multiple of the wide tile");
  dim3 grid(p.N / (32 * NB * WV), ceil_div(p.M, 32 * FM), p.splits), block(64 * WV);
  if constexpr (K2ORD) {  // the two-group kernel's default epilogue only
    BARK_REQUIRE(epi == Epi::Silu && fmt != 2, "gemm: no two-group-order wide kernel for this epilogue");
    if (fmt == 0) BARK_LAUNCH((gemm_wide_kernel<FM, false, false, false, (int)Epi::Silu, WV, true>), grid, block, 0, s, p);
    else BARK_LAUNCH((gemm_wide_kernel<FM, true, true, false, (int)Epi::Silu, WV, true>), grid, block, 0, s, p);
    return;
  }
#define BARK_K(L4, SW, AB, E) \
  BARK_LAUNCH((gemm_wide_kernel<FM, L4, SW, AB, (int)Epi::E, WV, false, NB>), grid, block, 0, s, p)
#define BARK_CASE(E)                                   \
  case Epi::E:                                         \
    if (fmt == 0) BARK_K(false, false, false, E);      \
    else BARK_K(true, true, false, E);                 \
    return;
#define BARK_PLAIN(E)                                  \
  case Epi::E:                                         \
    if (abf16) BARK_K(true, false, true, E);           \
    else BARK_K(true, false, false, E);                \
    return;
  if (fmt == 2) {
    switch (epi) {
      BARK_PLAIN(StoreF32)
      BARK_PLAIN(StoreF16)
      BARK_PLAIN(StoreBF16)
      default:
        break;
    }
  } else if constexpr (NB == 1) {  // one column block per wave: the epilogues tall_supported names
    switch (epi) {
      BARK_CASE(StoreF32)
      BARK_CASE(Qkv)
      default:
        break;
    }
  } else {
    switch (epi) {
      BARK_CASE(StoreF32)
      BARK_CASE(Silu)
      BARK_CASE(Glu)
      BARK_CASE(Qkv)
      BARK_CASE(RelK)
      BARK_CASE(BiasReluF16)
      BARK_CASE(FlattenReluF16)
      default:
        break;
    }
  }
#undef BARK_PLAIN
#undef BARK_CASE
#undef BARK_K
  throw Error{"gemm: no wide kernel for this epilogue and weight format"};
}

// The two-group kernel's instances: the encoder's epilogues on f16 weights
// (fmt 0) and on swizzled 4-bit weights (fmt 1) — the same kernel for both, so
// equal weight values give equal results; plain stores on plain 4-bit codes
// (fmt 2) with f16 or bf16 activations (the isolated linear).
bool k2_supported(Epi epi, int fmt) {
  if (fmt == 2) return epi == Epi::StoreF32 || epi == Epi::StoreF16 || epi == Epi::StoreBF16;
  switch (epi) {
    case Epi::StoreF32:
    case Epi::Silu:
    case Epi::Glu:
    case Epi::Qkv:
    case Epi::RelK:
      return true;
    default:
      return false;
  }
}

template <int FM, int EPI, bool L4, bool SW, bool AB>
void launch_k2_one(const GemmParams& p, hipStream_t s) {
  auto kern = gemm_k2_kernel<FM, L4, SW, AB, EPI>;
  constexpr size_t lds = K2Shape<FM, L4>::LDS;
  static_assert(lds <= 160 * 1024, "LDS budget");
  static const bool attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess;
  BARK_REQUIRE(attr, "gemm: cannot reserve LDS for the two-group kernel");
  dim3 grid(p.N / 256, ceil_div(p.M, 32 * FM), p.splits), block(512);
  BARK_LAUNCH(kern, grid, block, lds, s, p);
}

template <int FM>
void launch_k2(const GemmParams& p, Epi epi, int fmt, bool abf16, hipStream_t s) {
#define BARK_KE(E)                                                      \
  case Epi::E:                                                          \
    if (fmt == 1) launch_k2_one<FM, (int)Epi::E, true, true, false>(p, s);   \
    else launch_k2_one<FM, (int)Epi::E, false, false, false>(p, s);         \
    return;
#define BARK_KP(E)                                                      \
  case Epi::E:                                                          \
    if constexpr (FM <= 4) {                                            \
      if (abf16) {                                                      \
        launch_k2_one<FM, (int)Epi::E, true, false, true>(p, s);        \
        return;                                                         \
      }                                                                 \
    }                                                                   \
    launch_k2_one<FM, (int)Epi::E, true, false, false>(p, s);           \
    return;
  if (fmt == 2) {
    switch (epi) {
      BARK_KP(StoreF32)
      BARK_KP(StoreF16)
      BARK_KP(StoreBF16)
      default:
        break;
    }
  } else {
    switch (epi) {
      BARK_KE(StoreF32)
      BARK_KE(Silu)
      BARK_KE(Glu)
      BARK_KE(Qkv)
      BARK_KE(RelK)
      default:
        break;
    }
  }
#undef BARK_KE
#undef BARK_KP
  throw Error{"gemm: no two-group kernel for this epilogue and weight format"};
}

// Whether an epilogue runs on the two-group kernel by default. Measured on
// MI355X at T = 2207 (encoder step, per-op events): the FFN up projection
// (SiLU, N = 4096) is 3-9 % faster; the other linears are within a few
// percent either way, where the end-of-kernel store burst and the k-loop
// overhead bound both kernels alike, so they stay on gemm_wide_kernel. The
// choice depends on the epilogue only, so a weight's 4-bit and f16 forms
// always run the same kernel. BARK_HIP_GEMM_K2 = 1 uses it for every
// supported epilogue.
bool k2_default(Epi epi) {
  static const int forced = [] {
    const char* e = getenv("BARK_HIP_GEMM_K2");
    return e ? atoi(e) : -1;
  }();
  if (forced >= 1) return true;
  if (forced == 0) return false;
  return epi == Epi::Silu;
}

// Tile height (32-row blocks) of the two-group kernel: the height whose tile
// count fills the 256 CUs best (one workgroup per CU), taller on ties.
// BARK_HIP_GEMM_K2 = 0 disables the kernel, 3/4/5 forces a height.
int pick_k2_fm(int M, int N, int splits) {
  static const int forced = [] {
    const char* e = getenv("BARK_HIP_GEMM_K2");
    return e ? atoi(e) : -1;
  }();
  if (forced == 0) return 0;
  if (forced >= 3 && forced <= 5) return forced;
  constexpr int CUS = 256;
  int best = 4;
  double best_score = -1.0;
  const int fms[3] = {3, 4, 5};
  const double rate[3] = {0.95, 1.0, 1.05};
  for (int i = 0; i < 3; ++i) {
    const long tiles = (long)ceil_div(M, 32 * fms[i]) * (N / 256) * splits;
    const long rounds = (tiles + CUS - 1) / CUS;
    const double score = (double)tiles / (double)(CUS * rounds) * rate[i];
    if (score > best_score + 1e-9) {
      best_score = score;
      best = fms[i];
    }
  }
  return best;
}

void launch_k2_fm(int fm, const GemmParams& p, Epi epi, int fmt, bool abf16, hipStream_t s) {
  if (fm == 5 && !abf16) launch_k2<5>(p, epi, fmt, abf16, s);
  else if (fm == 3) launch_k2<3>(p, epi, fmt, abf16, s);
  else launch_k2<4>(p, epi, fmt, abf16, s);
}

// Full epilogue set: f16 weights and swizzled 4-bit weights (the encoder).
template <int BM, bool LUT4, bool SWZ>
void launch_full(const GemmParams& p, Epi epi, hipStream_t s) {
  dim3 grid(p.N / BN, ceil_div(p.M, BM)), block(256);
  switch (epi) {
#define BARK_CASE(E)                                                                          \
  case Epi::E:                                                                                \
    BARK_LAUNCH((gemm_kernel<BM, LUT4, SWZ, false, (int)Epi::E>), grid, block, 0, s, p); \
    break;
    BARK_CASE(StoreF32)
    BARK_CASE(StoreF16)
    BARK_CASE(StoreBF16)
    BARK_CASE(Silu)
    BARK_CASE(Resid)
    BARK_CASE(ResidHalf)
    BARK_CASE(Glu)
    BARK_CASE(Qkv)
    BARK_CASE(RelK)
    BARK_CASE(BiasReluF16)
    BARK_CASE(FlattenReluF16)
#undef BARK_CASE
  }
}

// Plain-layout 4-bit weights (the isolated linear): plain stores, f16 or bf16 A.
template <int BM>
void launch_plain(const GemmParams& p, Epi epi, bool abf16, hipStream_t s) {
  dim3 grid(p.N / BN, ceil_div(p.M, BM)), block(256);
#define BARK_CASE(E)                                                                              \
  case Epi::E:                                                                                    \
    if (abf16)                                                                                    \
      BARK_LAUNCH((gemm_kernel<BM, true, false, true, (int)Epi::E>), grid, block, 0, s, p);  \
    else                                                                                          \
      BARK_LAUNCH((gemm_kernel<BM, true, false, false, (int)Epi::E>), grid, block, 0, s, p); \
    break;
  switch (epi) {
    BARK_CASE(StoreF32)
    BARK_CASE(StoreF16)
    BARK_CASE(StoreBF16)
    default:
      throw Error{"gemm: plain-layout 4-bit weights support plain stores only"};
  }
#undef BARK_CASE
}

// 32-row MFMA blocks per wide tile (0 = use the 128-column kernel). Taller
// tiles spend fewer code expansions per MFMA but make fewer workgroups, so
// each height is scored as (fraction of the CU slots its launch keeps busy,
// counting every round) x (its relative per-CU rate); the best score wins.
// Two-block tiles run two workgroups per CU once there are more than one per
// CU. Rates and the short-K rule are from sweeps of the encoder shapes on
// MI355X. BARK_HIP_GEMM_WIDE = 0/2/3/4/5/6/8 forces a choice.
int pick_wide_fm(int M, int N, int K, int splits = 1, int max_fm = 8) {
  static const int forced = [] {
    const char* e = getenv("BARK_HIP_GEMM_WIDE");
    return e ? atoi(e) : -1;
  }();
  if (forced == 0 || (forced >= 2 && forced <= 6) || forced == 8) return forced;
  constexpr int CUS = 256;
  // a few k-tiles: the prologue dominates (measured: 3 blocks for the K = 256
  // front-end pointwise GEMMs, 2 for split-K chunks of 256)
  if (K / splits <= 256) return splits == 1 ? 3 : 2;
  int best = 2;
  double best_score = -1.0;
  const int fms[6] = {2, 3, 4, 5, 6, 8};
  const double rate[6] = {0.9, 0.95, 1.0, 1.05, 1.1, 1.15};
  for (int i = 0; i < 6; ++i) {
    if (fms[i] > max_fm) break;
    const long tiles = (long)ceil_div(M, 32 * fms[i]) * (N / 256) * splits;
    const long slots = (fms[i] == 2 && tiles > CUS) ? 2 * CUS : CUS;
    const long rounds = (tiles + slots - 1) / slots;
    const double score = (double)tiles / (double)(slots * rounds) * rate[i];
    if (score > best_score + 1e-9) {
      best_score = score;
      best = fms[i];
    }
  }
  return best;
}

// Short inputs (a few row tiles): one-wave workgroups of 32 or 64 rows x 64
// columns, which give 4x the workgroups of the four-wave tiles. Chosen when
// the four-wave tiles of 64 rows would fill fewer than half the CUs; the
// height is the one with more workgroups unless they would exceed four per
// CU. Returns 0 (use the four-wave tiles) or the height in row blocks (1, 2).
// BARK_HIP_GEMM_NARROW = 0/1/2 forces it off or a height.
int pick_narrow_fm(int M, int N, int splits) {
  static const int forced = [] {
    const char* e = getenv("BARK_HIP_GEMM_NARROW");
    return e ? atoi(e) : -1;
  }();
  if (forced >= 0 && forced <= 2) return forced;
  if (N % 64 != 0) return 0;
  const long wide_tiles = (long)ceil_div(M, 64) * (N / 256) * splits;
  if (wide_tiles >= 128) return 0;
  return (long)ceil_div(M, 32) * (N / 64) * splits <= 1024 ? 1 : 2;
}

// Column-strip kernel launches: NB 32-column blocks per workgroup (one, see
// strip_waves), MW waves of 32 rows each (2..8). f16 weights (fmt 0) and
// swizzled 4-bit weights (fmt 1).
template <int NB, bool K2ORD>
void launch_strip(const GemmParams& p, Epi epi, int fmt, int mw, hipStream_t s) {
  BARK_REQUIRE(mw >= 2 && mw <= 8 && p.N % (32 * NB) == 0 && fmt != 2, "gemm: bad strip launch");
  dim3 grid(p.N / (32 * NB), ceil_div(p.M, 32 * mw), p.splits), block(64 * mw);
#define BARK_SK(E)                                                                                         \
  do {                                                                                                     \
    if (fmt == 0) BARK_LAUNCH((gemm_strip_kernel<false, (int)Epi::E, NB, K2ORD>), grid, block, 0, s, p); \
    else BARK_LAUNCH((gemm_strip_kernel<true, (int)Epi::E, NB, K2ORD>), grid, block, 0, s, p);          \
  } while (0)
  if constexpr (K2ORD) {
    BARK_REQUIRE(epi == Epi::Silu, "gemm: no two-chain strip kernel for this epilogue");
    BARK_SK(Silu);
  } else {
    switch (epi) {
      case Epi::StoreF32: BARK_SK(StoreF32); break;
      case Epi::Silu: BARK_SK(Silu); break;
      case Epi::Qkv: BARK_SK(Qkv); break;
      default: throw Error{"gemm: no strip kernel for this epilogue"};
    }
  }
#undef BARK_SK
}

// Waves per strip workgroup (0: the strip kernel does not apply), for
// 33 <= M <= 256: one wave per 32-row block of a row tile, with the rows cut
// into as many equal tiles (of two blocks or more) as keep the launch within
// one workgroup per CU: more tiles fill more CUs, each tile making its own
// weight fragments. BARK_HIP_GEMM_STRIP = 0 turns the kernel off.
int strip_waves(int M, int N, int splits, Epi epi, int fmt) {
  static const int forced = [] {
    const char* e = getenv("BARK_HIP_GEMM_STRIP");
    return e ? atoi(e) : -1;
  }();
  if (forced == 0 || fmt == 2 || M <= 32 || M > 256) return 0;
  // GLU needs both halves of a pair in one wave (two column blocks): its
  // strips are too few to fill the CUs (measured slower than the one-wave
  // tiles at T = 188), so it stays there
  if (epi != Epi::StoreF32 && epi != Epi::Silu && epi != Epi::Qkv) return 0;
  // (measured on MI355X at T = 188: strips of two column blocks, which halve
  // the activation re-reads, ran 1.3-1.5x slower; allowing two workgroups per
  // CU, 512 per launch, 3 % slower)
  const long strips = (long)(N / 32) * splits;
  const int rb = ceil_div(M, 32);  // 32-row blocks
  int mw = rb < 2 ? 2 : rb;
  for (int rt = 2; rt <= rb / 2; ++rt)  // row tiles of at least two blocks
    if ((long)rt * strips <= 256) mw = ceil_div(rb, rt);
  return mw;
}

void launch_strip_for(const GemmParams& p, Epi epi, int fmt, int mw, bool k2ord, hipStream_t s) {
  if (k2ord) launch_strip<1, true>(p, epi, fmt, mw, s);
  else launch_strip<1, false>(p, epi, fmt, mw, s);
}

// Eight-wave tiles (128 x 256, each wave 128 rows x one 32-column block):
// where the 128-row tiles of a launch fit the 256 CUs in one round (and fill
// at least half of them), a workgroup per CU with two waves per SIMD beats the
// four-wave tiles, whose workgroups then sit one wave per SIMD. Measured on
// MI355X at T = 2207 (per launch): qkv 27.2 -> 22.9 us, FFN down 29.7 ->
// 28.3, the K = 1024 residual linears 15.7 -> 13.9-14.1. Per-element order
// is the wide kernel's (one chain per element), so results do not change.
// BARK_HIP_GEMM_TALL = 0 turns it off.
bool tall_enabled() {
  static const bool on = [] {
    const char* e = getenv("BARK_HIP_GEMM_TALL");
    return !(e && atoi(e) == 0);
  }();
  return on;
}

bool tall_fits(int M, int N, int splits) {
  if (!tall_enabled() || N % 256 != 0) return false;
  const long tiles = (long)ceil_div(M, 128) * (N / 256) * splits;
  return tiles >= 128 && tiles <= 256;
}

bool tall_supported(Epi epi, int fmt) {
  if (fmt == 2) return epi == Epi::StoreF32 || epi == Epi::StoreF16 || epi == Epi::StoreBF16;
  return epi == Epi::StoreF32 || epi == Epi::Qkv;
}

void launch_fm(int fm, int narrow, const GemmParams& p, Epi epi, int fmt, bool a_bf16, hipStream_t stream,
               bool k2ord = false) {
  if (narrow >= 1 && k2ord) launch_wide<1, 1, true>(p, epi, fmt, a_bf16, stream);
  else if (narrow == 1) launch_wide<1, 1>(p, epi, fmt, a_bf16, stream);
  else if (narrow == 2) launch_wide<2, 1>(p, epi, fmt, a_bf16, stream);
  else if (fm == 8) launch_wide<8>(p, epi, fmt, a_bf16, stream);
  else if (fm == 6) launch_wide<6>(p, epi, fmt, a_bf16, stream);
  else if (fm == 5) launch_wide<5>(p, epi, fmt, a_bf16, stream);
  else if (fm == 4) launch_wide<4>(p, epi, fmt, a_bf16, stream);
  else if (fm == 3) launch_wide<3>(p, epi, fmt, a_bf16, stream);
  else launch_wide<2>(p, epi, fmt, a_bf16, stream);
}

}  // namespace

void swizzle_codes(uint8_t* codes, size_t nbytes) {
  // plain byte j of a 4-byte group = n(2j) | n(2j+1) << 4; swizzled byte i = n(i) | n(i+4) << 4
  for (size_t g = 0; g + 4 <= nbytes; g += 4) {
    uint8_t n[8];
    for (int j = 0; j < 4; ++j) {
      n[2 * j] = codes[g + j] & 15;
      n[2 * j + 1] = codes[g + j] >> 4;
    }
    for (int i = 0; i < 4; ++i) codes[g + i] = (uint8_t)(n[i] | (n[i + 4] << 4));
  }
}

void gemm(const half* A, int lda, int M, const GemmWeight& W, Epi epi, const EpiArgs& ea,
          hipStream_t stream, bool a_bf16) {
  BARK_REQUIRE(A != nullptr, "gemm: null A");
  BARK_REQUIRE(W.k % (4 * BK) == 0 && W.k > 0, "gemm: K must be a positive multiple of 256");
  BARK_REQUIRE(W.n % BN == 0 && W.n > 0, "gemm: N must be a positive multiple of 128");
  BARK_REQUIRE(M > 0, "gemm: M must be positive");
  BARK_REQUIRE(lda >= W.k && lda % 8 == 0, "gemm: lda must be >= K and a multiple of 8");
  BARK_REQUIRE(W.lut4() ? (W.lut != nullptr) : (W.w16 != nullptr), "gemm: weight not set");
  GemmParams p{A, lda, W.w16, W.codes, W.lut, M, W.n, W.k, ea, 1, 0};
  BARK_REQUIRE(!a_bf16 || (W.lut4() && !W.swizzled), "gemm: bf16 activations need plain 4-bit weights");
  const bool fits32 = (double)M * lda * 2 < 4.0e9 && (double)W.n * W.k * 2 < 4.0e9;
  const int fmt = !W.lut4() ? 0 : W.swizzled ? 1 : 2;
  // short inputs: one-wave tiles, in the two-group kernel's summation order
  // where that kernel is the default (Silu), so results match longer inputs
  const bool k2 = W.n % 256 == 0 && fits32 && W.k / BK >= 4 && k2_supported(epi, fmt) && k2_default(epi);
  const int narrow = W.n % 256 == 0 && fits32 && wide_supported(epi, fmt) && (!k2 || epi == Epi::Silu)
                         ? pick_narrow_fm(M, W.n, 1)
                         : 0;
  const int mw = W.n % 256 == 0 && fits32 ? strip_waves(M, W.n, 1, epi, fmt) : 0;
  if (mw) {  // short inputs: weight fragments made once per workgroup
    launch_strip_for(p, epi, fmt, mw, k2 && epi == Epi::Silu, stream);
    BARK_HIP_CHECK(hipGetLastError());
    return;
  }
  if (!narrow && !k2 && fits32 && tall_supported(epi, fmt) && tall_fits(M, W.n, 1)) {
    launch_wide<4, 8, false, 1>(p, epi, fmt, a_bf16, stream);
    BARK_HIP_CHECK(hipGetLastError());
    return;
  }
  if (narrow) {  // the two-chain order at 64 rows spills: one row block there
    launch_fm(0, k2 ? 1 : narrow, p, epi, fmt, a_bf16, stream, k2);
    BARK_HIP_CHECK(hipGetLastError());
    return;
  }
  if (k2) {
    const int fm2 = pick_k2_fm(M, W.n, 1);
    if (fm2) {
      launch_k2_fm(fm2, p, epi, fmt, a_bf16, stream);
      BARK_HIP_CHECK(hipGetLastError());
      return;
    }
  }
  // the qkv epilogue spills heavily above four row blocks (0.9-1.3 KB per
  // lane, 30-80x slower launches), so its tiles stop at 128 rows
  const int max_fm = epi == Epi::Qkv ? 4 : 8;
  const int fm = W.n % 256 == 0 && fits32 && wide_supported(epi, fmt) ? pick_wide_fm(M, W.n, W.k, 1, max_fm) : 0;
  if (fm) {
    launch_fm(fm, 0, p, epi, fmt, a_bf16, stream);
    BARK_HIP_CHECK(hipGetLastError());
    return;
  }
  // N % 256 != 0 (the projector, narrow isolated linears) or an epilogue
  // without a wide instance: the 128-column kernel
  if (!W.lut4()) launch_full<64, false, false>(p, epi, stream);
  else if (W.swizzled) launch_full<64, true, true>(p, epi, stream);
  else launch_plain<64>(p, epi, a_bf16, stream);
  BARK_HIP_CHECK(hipGetLastError());
}

void gemm_split(const half* A, int lda, int M, const GemmWeight& W, int splits, float* part,
                int ldo, hipStream_t stream, bool a_bf16) {
  BARK_REQUIRE(A != nullptr && part != nullptr, "gemm_split: null operand");
  BARK_REQUIRE(splits >= 1 && W.k % (4 * BK) == 0 && W.k / (4 * BK) >= splits,
               "gemm_split: K must be a multiple of 256 with at least 256 per split");
  BARK_REQUIRE(W.n % 256 == 0 && W.n > 0, "gemm_split: N must be a positive multiple of 256");
  BARK_REQUIRE(M > 0 && ldo >= W.n, "gemm_split: bad M or ldo");
  BARK_REQUIRE(lda >= W.k && lda % 8 == 0, "gemm_split: lda must be >= K and a multiple of 8");
  BARK_REQUIRE(W.lut4() ? (W.lut != nullptr) : (W.w16 != nullptr), "gemm_split: weight not set");
  BARK_REQUIRE(!a_bf16 || (W.lut4() && !W.swizzled), "gemm_split: bf16 activations need plain 4-bit weights");
  BARK_REQUIRE((double)M * lda * 2 < 4.0e9 && (double)W.n * W.k * 2 < 4.0e9,
               "gemm_split: operand too large for 32-bit offsets");
  EpiArgs ea;
  ea.out_f32 = part;
  ea.ldo = ldo;
  GemmParams p{A, lda, W.w16, W.codes, W.lut, M, W.n, W.k, ea, splits, (size_t)M * ldo};
  const int fmt = !W.lut4() ? 0 : W.swizzled ? 1 : 2;
  const int narrow = k2_default(Epi::StoreF32) ? 0 : pick_narrow_fm(M, W.n, splits);
  const int mw = strip_waves(M, W.n, splits, Epi::StoreF32, fmt);
  if (mw) {
    launch_strip_for(p, Epi::StoreF32, fmt, mw, false, stream);
    BARK_HIP_CHECK(hipGetLastError());
    return;
  }
  if (!narrow && !k2_default(Epi::StoreF32) && tall_supported(Epi::StoreF32, fmt) && tall_fits(M, W.n, splits)) {
    launch_wide<4, 8, false, 1>(p, Epi::StoreF32, fmt, a_bf16, stream);
    BARK_HIP_CHECK(hipGetLastError());
    return;
  }
  if (k2_default(Epi::StoreF32)) {
    const int fm2 = pick_k2_fm(M, W.n, splits);
    if (fm2) {
      launch_k2_fm(fm2, p, Epi::StoreF32, fmt, a_bf16, stream);
      BARK_HIP_CHECK(hipGetLastError());
      return;
    }
  }
  int fm = pick_wide_fm(M, W.n, W.k, splits);
  if (fm == 0) fm = 2;
  launch_fm(fm, narrow, p, Epi::StoreF32, fmt, a_bf16, stream);
  BARK_HIP_CHECK(hipGetLastError());
}

// From a sweep of the N = 1024 residual linears at T = 2207 on MI355X.
// BARK_HIP_SPLIT_K1 / BARK_HIP_SPLIT_K4 override the count for K = 1024 /
// K = 4096.
int residual_splits(int n, int k) {
  static const int f1 = [] {
    const char* e = getenv("BARK_HIP_SPLIT_K1");
    return e ? atoi(e) : 0;
  }();
  static const int f4 = [] {
    const char* e = getenv("BARK_HIP_SPLIT_K4");
    return e ? atoi(e) : 0;
  }();
  int s = 1;
  if (n == 1024 && k == 1024) s = f1 ? f1 : 2;
  if (n == 1024 && k == 4096) s = f4 ? f4 : 3;  // 6 + 5 + 5 units: 216 tiles of 128 rows at T = 2207
  while (s > 1 && (k % 256 != 0 || k / 256 < s)) --s;
  return s;
}

namespace {
// Partial-sum workspace of the isolated linear, one per (device, stream):
// grow-only, freed at process exit.
float* isolated_workspace(hipStream_t stream, size_t bytes) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, std::pair<void*, size_t>> bufs;
  int dev = 0;
  BARK_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(mu);
  auto& b = bufs[{dev, stream}];
  if (b.second < bytes) {
    BARK_HIP_CHECK(hipStreamSynchronize(stream));  // earlier calls may still read the old one
    if (b.first) BARK_HIP_CHECK(hipFree(b.first));
    b.first = nullptr;
    b.second = 0;
    BARK_HIP_CHECK(hipMalloc(&b.first, bytes));
    b.second = bytes;
  }
  return static_cast<float*>(b.first);
}
}  // namespace

namespace {
// Partial sums of the no-allocation isolated linear: a file-scope device
// array, one copy per GPU (each GPU the library runs on holds it until the
// process ends). Host code must never hand its name to a kernel: in host code
// it is a stand-in, not a device address; scratch_ptr() looks up the real one.
static __device__ __align__(256) float scratch[ISOLATED_SCRATCH_BYTES / sizeof(float)];

// Device address of `scratch` on the current device, looked up once per
// device with hipGetSymbolAddress while that device is current; later calls
// reuse it. No allocation is involved (a fixed table, no containers).
float* scratch_ptr() {
  constexpr int MAX_DEVICES = 64;
  static std::mutex mu;
  static float* ptrs[MAX_DEVICES] = {};
  int dev = 0;
  BARK_HIP_CHECK(hipGetDevice(&dev));
  BARK_REQUIRE(dev >= 0 && dev < MAX_DEVICES, "scratch: device index out of range");
  std::lock_guard<std::mutex> lk(mu);
  if (!ptrs[dev]) {
    void* ptr = nullptr;
    BARK_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    BARK_REQUIRE(ptr != nullptr, "scratch: no device address");
    ptrs[dev] = static_cast<float*>(ptr);
  }
  return ptrs[dev];
}

// K splits of the isolated linear: split K when the output tiles alone leave
// most CUs idle, at small T as far as the CUs fill, and in two for a long K
// whose 128-row tiles cover fewer than half of them (T = 2207, K = 4096,
// N = 1024). A function of (M, N, K) only.
int isolated_splits(int M, const GemmWeight& W) {
  const long base = (long)ceil_div(M, 64) * (W.n / 256);
  int splits = 1;
  if (W.n % 256 == 0 && base < 128) {
    while (splits * 2 * base <= 256 && W.k % (splits * 2) == 0 && (W.k / (splits * 2)) % 256 == 0) splits *= 2;
  } else if (W.n % 256 == 0 && W.k >= 2048 && W.k % 512 == 0 && (long)ceil_div(M, 128) * (W.n / 256) < 128) {
    splits = 2;
  }
  return splits;
}

// The isolated linear with its partial sums in `part` (bytes available:
// part_bytes), or in the grow-only per-stream workspace when part is null.
// The skinny kernel for M <= 256 (plain 4-bit weights), else the wide
// kernels, with K split into partial sums in `part` (bytes available:
// part_bytes), or in the grow-only per-stream workspace when part is null,
// and one pass adding them in order.
void isolated_with(const half* A, int M, const GemmWeight& W, void* C, int c_kind, hipStream_t stream,
                   bool a_bf16, float* part, size_t part_bytes) {
  BARK_REQUIRE(c_kind >= 0 && c_kind <= 2, "gemm_isolated: bad output kind");
  const int mb = W.lut4() && !W.swizzled ? skinny_mb(M, W.n, W.k) : 0;
  if (mb > 0) {
    BARK_REQUIRE(A != nullptr && W.lut != nullptr && C != nullptr, "gemm_isolated: null operand");
    BARK_REQUIRE((size_t)W.n * W.k / 2 < (1ull << 31) && (size_t)M * W.k < (1ull << 31),
                 "gemm_isolated: operand too large");
    SkinnyArgs a;
    a.p.A = A;
    a.p.lda = W.k;
    a.p.codes = W.codes;
    a.p.lut = W.lut;
    a.p.M = M;
    a.p.N = W.n;
    a.p.K = W.k;
    a.out = C;
    a.out_kind = c_kind;
    if (mb == 1) launch_skinny_mb<1>(a, a_bf16, stream);
    else if (mb == 2) launch_skinny_mb<2>(a, a_bf16, stream);
    else if (mb == 3) launch_skinny_mb<3>(a, a_bf16, stream);
    else launch_skinny_mb<4>(a, a_bf16, stream);
    BARK_HIP_CHECK(hipGetLastError());
    return;
  }
  const int splits = isolated_splits(M, W);
  if (splits == 1) {
    EpiArgs e;
    e.ldo = W.n;
    Epi epi = Epi::StoreF32;
    if (c_kind == 0) {
      e.out_f32 = static_cast<float*>(C);
    } else {
      e.out_f16 = static_cast<half*>(C);
      epi = c_kind == 1 ? Epi::StoreF16 : Epi::StoreBF16;
    }
    gemm(A, W.k, M, W, epi, e, stream, a_bf16);
    return;
  }
  // the chunks' partial sums go to the workspace and one pass adds them in order
  const size_t stride = (size_t)M * W.n;
  const size_t need = splits * stride * sizeof(float);
  if (part) {
    BARK_REQUIRE(need <= part_bytes,
                 "T x N too large for the fixed scratch of the no-allocation linear: it needs " +
                     std::to_string(need) + " bytes of partial sums, the limit is " + std::to_string(part_bytes) +
                     " (use bark_hip_lowbit_linear)");
  } else {
    part = isolated_workspace(stream, need);
  }
  gemm_split(A, W.k, M, W, splits, part, W.n, stream, a_bf16);
  const long n4 = (long)(stride / 4);
  BARK_LAUNCH(split_reduce_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream, part,
                     splits, stride, C, c_kind, n4);
  BARK_HIP_CHECK(hipGetLastError());
}
}  // namespace

void gemm_isolated(const half* A, int M, const GemmWeight& W, void* C, int c_kind, hipStream_t stream,
                   bool a_bf16) {
  isolated_with(A, M, W, C, c_kind, stream, a_bf16, nullptr, 0);
}

void gemm_isolated_noalloc(const half* A, int M, const GemmWeight& W, void* C, int c_kind, hipStream_t stream,
                           bool a_bf16) {
  isolated_with(A, M, W, C, c_kind, stream, a_bf16, scratch_ptr(), ISOLATED_SCRATCH_BYTES);
}


}  // namespace bark
