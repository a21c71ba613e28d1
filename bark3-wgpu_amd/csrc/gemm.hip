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
// thread streams 16 bytes of codes (32 weights of one row) per k-tile with one
// coalesced load, expands them through the row's table (held in LDS) and
// writes the f16 values into the B tile, so every weight is expanded once per
// workgroup and reused by all BM rows.
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
};

template <int EPI>
__device__ inline void store_one(const EpiArgs& ea, int r, int c, float v) {
  if constexpr (EPI == (int)Epi::StoreF32) {
    if (ea.bias) v += ea.bias[c];
    ea.out_f32[(size_t)r * ea.ldo + c] = v;
  } else if constexpr (EPI == (int)Epi::StoreF16) {
    if (ea.bias) v += ea.bias[c];
    ea.out_f16[(size_t)r * ea.ldo + c] = (half)v;
  } else if constexpr (EPI == (int)Epi::StoreBF16) {
    if (ea.bias) v += ea.bias[c];
    uint32_t u = __float_as_uint(v);
    u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even (finite inputs)
    reinterpret_cast<uint16_t*>(ea.out_f16)[(size_t)r * ea.ldo + c] = (uint16_t)(u >> 16);
  } else if constexpr (EPI == (int)Epi::Silu) {
    ea.out_f16[(size_t)r * ea.ldo + c] = (half)silu(v);
  } else if constexpr (EPI == (int)Epi::Resid) {
    float* p = ea.out_f32 + (size_t)r * ea.ldo + c;
    *p = *p + ea.scale * v;
  } else if constexpr (EPI == (int)Epi::Qkv) {
    const int which = c >> 10, hd = c & 1023, h = hd >> 7, d = hd & 127;
    const size_t hr = ((size_t)h * ea.mp + r) * HDIM + d;
    if (which == 0) {
      ea.qu[hr] = (half)(v + ea.bu[hd]);
      ea.qv[hr] = (half)(v + ea.bv[hd]);
    } else if (which == 1) {
      ea.kh[hr] = (half)v;
    } else {
      ea.vt[((size_t)h * HDIM + d) * ea.mp + r] = (half)v;
    }
  } else if constexpr (EPI == (int)Epi::RelK) {
    const int h = c >> 7, d = c & 127;
    ea.rk[((size_t)h * ea.pp + r) * HDIM + d] = (half)v;
  } else if constexpr (EPI == (int)Epi::BiasReluF16) {
    v += ea.bias[c];
    ea.out_f16[(size_t)r * ea.ldo + c] = (half)(v > 0.0f ? v : 0.0f);
  } else if constexpr (EPI == (int)Epi::FlattenReluF16) {
    v += ea.bias[c];
    const int t = r >> 4, m = r & 15;
    ea.out_f16[(size_t)t * ea.ldo + c * 16 + m] = (half)(v > 0.0f ? v : 0.0f);
  }
}

template <int BM, bool LUT4, bool ABF16, int EPI>
__global__ void __launch_bounds__(256) gemm_kernel(GemmParams p) {
  constexpr int WTM = BM / 2;       // wave tile rows
  constexpr int FM = WTM / 32;      // 32-row MFMA blocks per wave
  constexpr int FN = 2;             // 32-col MFMA blocks per wave (64 cols)
  constexpr int A_CH = BM * BK / 8 / 256;  // 16-byte chunks of A per thread
  constexpr int B_CH = BN * BK / 8 / 256;  // (f16 mode)

  __shared__ __attribute__((aligned(16))) half As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) half Bs[2][BN * LDK];
  __shared__ __attribute__((aligned(16))) half lut_s[LUT4 ? BN * 16 : 8];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int l32 = lane & 31, lhi = lane >> 5;

  uint4 a_reg[A_CH];
  uint4 b_reg[LUT4 ? 1 : B_CH];

  if constexpr (LUT4) {
    // 128 rows x 16 halves = 256 chunks of 16 B: one per thread.
    const uint4* src = reinterpret_cast<const uint4*>(p.lut + (size_t)n0 * 16);
    reinterpret_cast<uint4*>(lut_s)[tid] = src[tid];
  }

  auto load_tiles = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int ch = tid + 256 * i, row = ch >> 3, col = (ch & 7) * 8;
      a_reg[i] = (m0 + row < p.M)
                     ? *reinterpret_cast<const uint4*>(p.A + (size_t)(m0 + row) * p.lda + k0 + col)
                     : uint4{0u, 0u, 0u, 0u};
    }
    if constexpr (LUT4) {
      const int row = tid >> 1, part = tid & 1;
      b_reg[0] = *reinterpret_cast<const uint4*>(p.codes + (size_t)(n0 + row) * (p.K >> 1) +
                                                 (k0 >> 1) + part * 16);
    } else {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int ch = tid + 256 * i, row = ch >> 3, col = (ch & 7) * 8;
        b_reg[i] = *reinterpret_cast<const uint4*>(p.W + (size_t)(n0 + row) * p.K + k0 + col);
      }
    }
  };

  auto store_tiles = [&](int stage) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int ch = tid + 256 * i, row = ch >> 3, col = (ch & 7) * 8;
      if constexpr (ABF16) {  // bf16 -> f16: exact for |x| in the f16 normal range
        const uint32_t w4[4] = {a_reg[i].x, a_reg[i].y, a_reg[i].z, a_reg[i].w};
        half8 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = (half)__uint_as_float(w4[e] << 16);
          v[2 * e + 1] = (half)__uint_as_float(w4[e] & 0xffff0000u);
        }
        st_half8(&As[stage][row * LDK + col], v);
      } else {
        *reinterpret_cast<uint4*>(&As[stage][row * LDK + col]) = a_reg[i];
      }
    }
    if constexpr (LUT4) {
      const int row = tid >> 1, part = tid & 1;
      const half* tb = lut_s + row * 16;
      const uint32_t w4[4] = {b_reg[0].x, b_reg[0].y, b_reg[0].z, b_reg[0].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t w = w4[q];  // 8 codes, low nibble first = ascending k
        half8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = tb[(w >> (4 * e)) & 15u];
        st_half8(&Bs[stage][row * LDK + part * 32 + q * 8], v);
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int ch = tid + 256 * i, row = ch >> 3, col = (ch & 7) * 8;
        *reinterpret_cast<uint4*>(&Bs[stage][row * LDK + col]) = b_reg[i];
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

  const int nk = p.K / BK;
  load_tiles(0);
  if constexpr (LUT4) __syncthreads();  // lut_s visible before expansion
  store_tiles(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tiles(kt + 1);
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
    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

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
        ea.out_f32[(size_t)r * ea.ldo + c] = a / (1.0f + __expf(-g));
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

template <int BM, bool LUT4>
void launch_bm(const GemmParams& p, Epi epi, bool abf16, hipStream_t s) {
  dim3 grid(p.N / BN, ceil_div(p.M, BM)), block(256);
  if (abf16) {
    switch (epi) {
      case Epi::StoreF32:
        hipLaunchKernelGGL((gemm_kernel<BM, LUT4, true, (int)Epi::StoreF32>), grid, block, 0, s, p);
        break;
      case Epi::StoreF16:
        hipLaunchKernelGGL((gemm_kernel<BM, LUT4, true, (int)Epi::StoreF16>), grid, block, 0, s, p);
        break;
      case Epi::StoreBF16:
        hipLaunchKernelGGL((gemm_kernel<BM, LUT4, true, (int)Epi::StoreBF16>), grid, block, 0, s, p);
        break;
      default:
        throw Error{"gemm: bf16 activations support plain stores only"};
    }
    return;
  }
  switch (epi) {
#define BARK_CASE(E)                                                                    \
  case Epi::E:                                                                          \
    hipLaunchKernelGGL((gemm_kernel<BM, LUT4, false, (int)Epi::E>), grid, block, 0, s, p); \
    break;
    BARK_CASE(StoreF32)
    BARK_CASE(StoreF16)
    BARK_CASE(StoreBF16)
    BARK_CASE(Silu)
    BARK_CASE(Resid)
    BARK_CASE(Glu)
    BARK_CASE(Qkv)
    BARK_CASE(RelK)
    BARK_CASE(BiasReluF16)
    BARK_CASE(FlattenReluF16)
#undef BARK_CASE
  }
}

}  // namespace

void gemm(const half* A, int lda, int M, const GemmWeight& W, Epi epi, const EpiArgs& ea,
          hipStream_t stream, bool a_bf16) {
  BARK_REQUIRE(A != nullptr, "gemm: null A");
  BARK_REQUIRE(W.k % BK == 0 && W.k > 0, "gemm: K must be a positive multiple of 64");
  BARK_REQUIRE(W.n % BN == 0 && W.n > 0, "gemm: N must be a positive multiple of 128");
  BARK_REQUIRE(M > 0, "gemm: M must be positive");
  BARK_REQUIRE(lda >= W.k && lda % 8 == 0, "gemm: lda must be >= K and a multiple of 8");
  BARK_REQUIRE(W.lut4() ? (W.lut != nullptr) : (W.w16 != nullptr), "gemm: weight not set");
  GemmParams p{A, lda, W.w16, W.codes, W.lut, M, W.n, W.k, ea};
  // Wide tiles when they still give about one workgroup per CU.
  const bool big = (long)ceil_div(M, 128) * (W.n / BN) >= 192;
  if (W.lut4()) {
    if (big) launch_bm<128, true>(p, epi, a_bf16, stream);
    else launch_bm<64, true>(p, epi, a_bf16, stream);
  } else {
    if (big) launch_bm<128, false>(p, epi, a_bf16, stream);
    else launch_bm<64, false>(p, epi, a_bf16, stream);
  }
  BARK_HIP_CHECK(hipGetLastError());
}

}  // namespace bark
