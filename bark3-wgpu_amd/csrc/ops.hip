// Row-wise and elementwise kernels of the encoder block and the conv front end.
// All are HBM-bound: each reads its input once and writes its output once.
#include "kernels.h"

namespace bark {
namespace {

// ---------------------------------------------------------------- LayerNorm --
// One wave per 1024-wide row; lane l holds columns 4l + 256i (i < 4) so every
// load is a coalesced float4. mean = E[x], var = E[x^2] - mean^2 and
// y = (x - mean) * (1/sqrt(var + 1e-5)) * w + b, the reference formula
// (src/encoder/shader_sources.rs:185-228, src/cpu/ops.rs:15-56).
// w and b of a lane's 16 columns, loaded before the row statistics need them
struct LnParams {
  float w[16], b[16];
  __device__ LnParams(const float* wp, const float* bp, int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 4 * lane + 256 * i;
      const floatx4 wv = *reinterpret_cast<const floatx4*>(wp + c);
      const floatx4 bv = *reinterpret_cast<const floatx4*>(bp + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) w[4 * i + e] = wv[e], b[4 * i + e] = bv[e];
    }
  }
};

__device__ inline void ln_row(float (&x)[16], const LnParams& prm) {
  float s = 0.0f, q = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    s += x[i];
    q += x[i] * x[i];
  }
  s = wave_sum(s);
  q = wave_sum(q);
  const float mean = s * (1.0f / 1024.0f);
  const float var = q * (1.0f / 1024.0f) - mean * mean;
  const float inv = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = (x[i] - mean) * inv * prm.w[i] + prm.b[i];
}

__device__ inline void load_row(const float* x, float (&v)[16], int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const floatx4 t = *reinterpret_cast<const floatx4*>(x + 4 * lane + 256 * i);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * i + e] = t[e];
  }
}

__device__ inline void store_row32(float* y, const float (&v)[16], int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const floatx4 t = {v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
    *reinterpret_cast<floatx4*>(y + 4 * lane + 256 * i) = t;
  }
}

__device__ inline void store_row16(half* y, const float (&v)[16], int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const half4 t = {(half)v[4 * i], (half)v[4 * i + 1], (half)v[4 * i + 2], (half)v[4 * i + 3]};
    *reinterpret_cast<half4*>(y + 4 * lane + 256 * i) = t;
  }
}

// x += scale * (p_0 + p_1 + ...), partial sums added in split order. Up to
// four splits have all their loads issued before the first add.
template <int S>
__device__ inline void add_residual_n(float (&v)[16], const ResidIn& res, size_t row_off, int lane) {
  float p[S][16];
#pragma unroll
  for (int s = 0; s < S; ++s) load_row(res.part + s * res.stride + row_off, p[s], lane);
#pragma unroll
  for (int s = 1; s < S; ++s)
#pragma unroll
    for (int i = 0; i < 16; ++i) p[0][i] += p[s][i];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = v[i] + res.scale * p[0][i];
}

__device__ inline void add_residual(float (&v)[16], const ResidIn& res, size_t row_off, int lane) {
  switch (res.splits) {
    case 1: add_residual_n<1>(v, res, row_off, lane); return;
    case 2: add_residual_n<2>(v, res, row_off, lane); return;
    case 3: add_residual_n<3>(v, res, row_off, lane); return;
    case 4: add_residual_n<4>(v, res, row_off, lane); return;
    default: break;
  }
  float p[16];
  load_row(res.part + row_off, p, lane);
  for (int s = 1; s < res.splits; ++s) {
    float q[16];
    load_row(res.part + s * res.stride + row_off, q, lane);
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] += q[i];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = v[i] + res.scale * p[i];
}

__global__ void __launch_bounds__(256) ln_kernel(float* x, const float* w, const float* b,
                                                 half* y16, float* y32, int rows, ResidIn res) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const LnParams prm(w, b, lane);
  float v[16];
  load_row(x + (size_t)r * HIDDEN, v, lane);
  if (res.splits) {
    add_residual(v, res, (size_t)r * HIDDEN, lane);
    store_row32(x + (size_t)r * HIDDEN, v, lane);
  }
  ln_row(v, prm);
  if (y32) store_row32(y32 + (size_t)r * HIDDEN, v, lane);
  if (y16) store_row16(y16 + (size_t)r * HIDDEN, v, lane);
}

__global__ void __launch_bounds__(256) resid_kernel(float* x, int rows, ResidIn res) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  float v[16];
  load_row(x + (size_t)r * HIDDEN, v, lane);
  add_residual(v, res, (size_t)r * HIDDEN, lane);
  store_row32(x + (size_t)r * HIDDEN, v, lane);
}

// Block-final norm_out of layer l fused with norm_feed_forward1 of layer l+1.
__global__ void __launch_bounds__(256) ln2_kernel(const float* x, const float* wa,
                                                  const float* ba, float* y32, const float* wb,
                                                  const float* bb, half* y16, int rows,
                                                  ResidIn res) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const LnParams pa(wa, ba, lane), pb(wb, bb, lane);
  float v[16];
  load_row(x + (size_t)r * HIDDEN, v, lane);
  if (res.splits) add_residual(v, res, (size_t)r * HIDDEN, lane);
  ln_row(v, pa);
  store_row32(y32 + (size_t)r * HIDDEN, v, lane);
  ln_row(v, pb);
  store_row16(y16 + (size_t)r * HIDDEN, v, lane);
}

// ------------------------------------------------- depthwise conv + BN + SiLU --
// y[t,c] = sum_{i<9} x[t+i-4, c] * w[c,i] over frames inside the row's
// sequence [start, end) (zero padding at the sequence edge, the length mask
// of src/encoder/shader_sources.rs:344-376 / src/cpu/ops.rs:195-233), then
// z = silu(y * a_c + b_c) with the folded BatchNorm; f32 multiply-adds in
// ascending tap order (fused; the reference CPU rounds the product first,
// a difference of an ulp per tap). A thread owns 4 consecutive channels
// (float4 loads) and DW_ROWS consecutive rows, reading its (DW_ROWS + 8)-row
// window once; a wave covers 256 channels, a workgroup 4 row groups. Row
// groups whose windows lie inside their sequences skip the tap masks. The
// weights are tap-major, one float4 per tap (36 scalar loads per thread in
// channel-major order cost 6 % of the kernel); 2 and 8 rows per thread
// measured slower than 4.
constexpr int DW_ROWS = 4;

__global__ void __launch_bounds__(256) dwconv_kernel(const float* g, const float* dw,
                                                     const float* bn_a, const float* bn_b,
                                                     const int2* bounds, half* out, int rows) {
  const int c = (blockIdx.y * 64 + (threadIdx.x & 63)) * 4;
  const int r0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + (threadIdx.x >> 6)) * DW_ROWS);
  if (r0 >= rows) return;
  float w[4][9];
#pragma unroll
  for (int i = 0; i < 9; ++i) {  // dw is tap-major [9][1024]
    const floatx4 t = *reinterpret_cast<const floatx4*>(dw + i * HIDDEN + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e][i] = t[e];
  }
  const floatx4 a = *reinterpret_cast<const floatx4*>(bn_a + c);
  const floatx4 b = *reinterpret_cast<const floatx4*>(bn_b + c);
  floatx4 win[DW_ROWS + 8];
#pragma unroll
  for (int i = 0; i < DW_ROWS + 8; ++i) {
    const int r = r0 - 4 + i;
    win[i] = (r >= 0 && r < rows) ? *reinterpret_cast<const floatx4*>(g + (size_t)r * HIDDEN + c)
                                  : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  int2 be[DW_ROWS];
  bool inside = r0 + DW_ROWS <= rows;
#pragma unroll
  for (int t = 0; t < DW_ROWS; ++t) {
    be[t] = bounds[min(r0 + t, rows - 1)];  // wave-uniform
    inside = inside && be[t].x <= r0 + t - 4 && r0 + t + 4 < be[t].y;
  }
  floatx4 y[DW_ROWS];
  if (inside) {
#pragma unroll
    for (int t = 0; t < DW_ROWS; ++t) {
      floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < 9; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = fmaf(win[t + i][e], w[e][i], acc[e]);
      y[t] = acc;
    }
  } else {
#pragma unroll
    for (int t = 0; t < DW_ROWS; ++t) {
      const int r = r0 + t;
      floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < 9; ++i) {
        const int rr = r + i - 4;
        if (rr >= be[t].x && rr < be[t].y) {
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[e] = fmaf(win[t + i][e], w[e][i], acc[e]);
        }
      }
      y[t] = acc;
    }
  }
#pragma unroll
  for (int t = 0; t < DW_ROWS; ++t) {
    const int r = r0 + t;
    if (r >= rows) break;
    half4 z;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = fmaf(y[t][e], a[e], b[e]);
      z[e] = (half)(v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)));
    }
    *reinterpret_cast<half4*>(out + (size_t)r * HIDDEN + c) = z;
  }
}

// ---------------------------------------------------------------- converts --
__global__ void f32_to_f16_kernel(const float* x, half* y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (half)x[i];
}

__global__ void f32_to_f16_rows_kernel(const float* x, int cols, half* y, int ldy, int rows) {
  const int r = blockIdx.y;
  for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += gridDim.x * blockDim.x)
    y[(size_t)r * ldy + c] = (half)x[(size_t)r * cols + c];
}

__global__ void copy_rows_kernel(const float* x, int ldx, float* y, int ldy, int cols) {
  const int r = blockIdx.y;
  for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += gridDim.x * blockDim.x)
    y[(size_t)r * ldy + c] = x[(size_t)r * ldx + c];
}

// -------------------------------------------------------------- front end --
// conv 1->256, 3x3, stride 2, pad 1, then ReLU (src/sub.rs:116-168), fused
// with the first depthwise 3x3 stride 2 (src/sub.rs:174-203): the conv1 map
// (8828 x 64 x 256 f16 = 289 MB at 17656 frames) never goes to HBM. A
// workgroup makes FD_ROWS output rows x 32 columns x FD_CH channels; it first
// computes the 2 * FD_ROWS + 1 conv1 rows they read into LDS, as the f16 value
// an unfused conv1 would store, then the depthwise sums from there. conv1 is
// b + w0*x0 + ... + w8*x8 in tap order as fused multiply-adds (the reference
// AXPY rounds each product first: an ulp per tap); conv1 rows >= vlen1 are
// zeroed (mask_time, src/sub.rs:288-300); the depthwise sum runs over the
// in-range taps in (ki, kj) order from its bias, and output rows >= vlen2 are
// zeroed. Thread = 4 consecutive channels x a strided set of positions.
constexpr int FD_ROWS = 4, FD_CH = 32;
constexpr int FD_C1R = 2 * FD_ROWS + 1;  // conv1 rows per workgroup
constexpr int FD_MELR = 2 * FD_C1R + 1;  // mel rows per workgroup

__global__ void __launch_bounds__(256) conv1_dw_kernel(const float* mel, int frames, int f1, int vlen1,
                                                       const float* w1, const float* b1, const float* wd,
                                                       const float* bd, half* out, int t2, int vlen2) {
  __shared__ float patch[FD_MELR][MEL + 2];  // columns -1 .. 128, zero outside the mel
  __shared__ __attribute__((aligned(16))) half c1[FD_C1R][64][FD_CH];
  const int r0 = blockIdx.x * FD_ROWS;  // first output row
  const int tid = threadIdx.x;
  const int ii0 = 2 * r0 - 1;           // first conv1 row
  const int mr0 = 2 * ii0 - 1;          // first mel row
  // every load of the patch is issued before its first LDS store (one wait
  // for memory, not one per element)
  constexpr int PATCH_N = FD_MELR * (MEL + 2), PATCH_IT = (PATCH_N + 255) / 256;
  float pv[PATCH_IT];
#pragma unroll
  for (int k = 0; k < PATCH_IT; ++k) {
    const int i = tid + 256 * k;
    const int r = i / (MEL + 2), ci = i % (MEL + 2);
    const int si = mr0 + r, sj = ci - 1;
    pv[k] = (i < PATCH_N && si >= 0 && si < frames && sj >= 0 && sj < MEL) ? mel[(size_t)si * MEL + sj] : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < PATCH_IT; ++k)
    if (tid + 256 * k < PATCH_N) (&patch[0][0])[tid + 256 * k] = pv[k];
  __syncthreads();
  const int cg = tid & 7, pg = tid >> 3;  // channel group (4 channels), position group
  const int cl = 4 * cg, c = blockIdx.y * FD_CH + cl;
  float w[4][9], bb[4];
  {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int t = 0; t < 9; ++t) w[e][t] = w1[(c + e) * 9 + t];
      bb[e] = b1[c + e];
    }
    for (int p = pg; p < FD_C1R * 64; p += 32) {
      const int lr = p >> 6, j = p & 63;
      const int ii = ii0 + lr;
      if (ii < 0 || ii >= f1) continue;  // rows the depthwise conv never reads
      float x[9];
#pragma unroll
      for (int t = 0; t < 9; ++t) x[t] = patch[2 * lr + t / 3][2 * j + t % 3];
      half4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float acc = bb[e];
#pragma unroll
        for (int t = 0; t < 9; ++t) acc = fmaf(w[e][t], x[t], acc);
        acc = acc > 0.0f ? acc : 0.0f;
        if (ii >= vlen1) acc = 0.0f;
        v[e] = (half)acc;
      }
      *reinterpret_cast<half4*>(&c1[lr][j][cl]) = v;
    }
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma unroll
    for (int t = 0; t < 9; ++t) w[e][t] = wd[(c + e) * 9 + t];
    bb[e] = bd[c + e];
  }
  for (int q = pg; q < FD_ROWS * 32; q += 32) {
    const int i2 = r0 + (q >> 5), j2 = q & 31;  // row uniform per iteration
    if (i2 >= t2) break;
    float sacc[4] = {bb[0], bb[1], bb[2], bb[3]};
#pragma unroll
    for (int ki = 0; ki < 3; ++ki) {
      const int ii = 2 * i2 + ki - 1;
      if (ii < 0 || ii >= f1) continue;
#pragma unroll
      for (int kj = 0; kj < 3; ++kj) {
        const int jj = 2 * j2 + kj - 1;
        if (jj < 0 || jj >= 64) continue;
        const half4 xv = *reinterpret_cast<const half4*>(&c1[ii - ii0][jj][cl]);
#pragma unroll
        for (int e = 0; e < 4; ++e) sacc[e] = fmaf(w[e][ki * 3 + kj], (float)xv[e], sacc[e]);
      }
    }
    half4 z;
#pragma unroll
    for (int e = 0; e < 4; ++e) z[e] = (half)(i2 >= vlen2 ? 0.0f : sacc[e]);
    *reinterpret_cast<half4*>(out + ((size_t)i2 * 32 + j2) * SUB_CH + c) = z;
  }
}

// depthwise 3x3 stride 2 pad 1 (src/sub.rs:174-203): s = b + sum w*x over the
// in-range taps in (ki, kj) order (fused multiply-adds); rows >= vlen zeroed. A thread computes 8
// consecutive channels of one output pixel with 16-byte loads; a workgroup
// covers 8 pixels per pass (32 threads x 8 channels = 256 channels each).
constexpr int DW2_PIX = 32;  // output pixels per workgroup

__global__ void __launch_bounds__(256) sub_dw_kernel(const half* in, int t_in, int m_in,
                                                     const float* w, const float* b, half* out,
                                                     int t_out, int m_out, int vlen) {
  const int c = (threadIdx.x & 31) * 8;
  float wr[8][9];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int t = 0; t < 9; ++t) wr[e][t] = w[(c + e) * 9 + t];
  float bias[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) bias[e] = b[c + e];
  const int npix = t_out * m_out;
  for (int p = threadIdx.x >> 5; p < DW2_PIX; p += 8) {
    const int pix = blockIdx.x * DW2_PIX + p;
    if (pix >= npix) break;
    const int i = pix / m_out, j = pix % m_out;
    // the nine taps' loads first (one wait for memory), then the sum over the
    // in-range taps in (ki, kj) order
    half8 xt[9];
    bool ok[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      const int ii = 2 * i + t / 3 - 1, jj = 2 * j + t % 3 - 1;
      ok[t] = ii >= 0 && ii < t_in && jj >= 0 && jj < m_in;
      xt[t] = ok[t] ? ld_half8(in + ((size_t)ii * m_in + jj) * SUB_CH + c) : half8{};
    }
    float s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = bias[e];
#pragma unroll
    for (int t = 0; t < 9; ++t) {
      if (!ok[t]) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] = fmaf(wr[e][t], (float)xt[t][e], s[e]);
    }
    half8 z;
#pragma unroll
    for (int e = 0; e < 8; ++e) z[e] = (half)(i >= vlen ? 0.0f : s[e]);
    st_half8(out + (size_t)pix * SUB_CH + c, z);
  }
}

}  // namespace

static void check_resid(const ResidIn& res) {
  BARK_REQUIRE(res.splits == 0 || (res.part != nullptr && res.splits > 0 && res.splits <= 16),
               "residual partials: bad split count or null buffer");
}

void layer_norm(float* x, const float* w, const float* b, half* y16, float* y32, int rows,
                hipStream_t stream, const ResidIn& res) {
  if (rows <= 0) return;
  check_resid(res);
  BARK_LAUNCH(ln_kernel, dim3(ceil_div(rows, 4)), dim3(256), 0, stream, x, w, b, y16,
                     y32, rows, res);
  BARK_HIP_CHECK(hipGetLastError());
}

void layer_norm2(const float* x, const float* wa, const float* ba, float* y32, const float* wb,
                 const float* bb, half* y16, int rows, hipStream_t stream, const ResidIn& res) {
  if (rows <= 0) return;
  check_resid(res);
  BARK_LAUNCH(ln2_kernel, dim3(ceil_div(rows, 4)), dim3(256), 0, stream, x, wa, ba,
                     y32, wb, bb, y16, rows, res);
  BARK_HIP_CHECK(hipGetLastError());
}

void apply_residual(float* x, int rows, const ResidIn& res, hipStream_t stream) {
  if (rows <= 0 || res.splits == 0) return;
  check_resid(res);
  BARK_LAUNCH(resid_kernel, dim3(ceil_div(rows, 4)), dim3(256), 0, stream, x, rows, res);
  BARK_HIP_CHECK(hipGetLastError());
}

void dwconv_bn_silu(const float* g, const float* dw, const float* bn_a, const float* bn_b,
                    const int2* bounds, half* out, int rows, hipStream_t stream) {
  if (rows <= 0) return;
  BARK_LAUNCH(dwconv_kernel, dim3(ceil_div(rows, 4 * DW_ROWS), HIDDEN / 256), dim3(256), 0,
                     stream, g, dw, bn_a, bn_b, bounds, out, rows);
  BARK_HIP_CHECK(hipGetLastError());
}

__global__ void __launch_bounds__(256) zero_fill_kernel(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) p[i] = uint4{0, 0, 0, 0};
}

void zero_fill(void* p, size_t bytes, hipStream_t stream) {
  BARK_REQUIRE(bytes % 16 == 0 && reinterpret_cast<uintptr_t>(p) % 16 == 0, "zero_fill: 16-byte units");
  const size_t n16 = bytes / 16;
  if (n16 == 0) return;
  BARK_LAUNCH(zero_fill_kernel, dim3((unsigned)std::min<size_t>((n16 + 255) / 256, 4096)), dim3(256), 0, stream,
              static_cast<uint4*>(p), n16);
  BARK_HIP_CHECK(hipGetLastError());
}

void f32_to_f16(const float* x, half* y, size_t n, hipStream_t stream) {
  if (n == 0) return;
  BARK_LAUNCH(f32_to_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     x, y, n);
  BARK_HIP_CHECK(hipGetLastError());
}

void f32_to_f16_rows(const float* x, int rows, int cols, half* y, int ldy, hipStream_t stream) {
  if (rows <= 0) return;
  BARK_LAUNCH(f32_to_f16_rows_kernel, dim3(ceil_div(cols, 256), rows), dim3(256), 0,
                     stream, x, cols, y, ldy, rows);
  BARK_HIP_CHECK(hipGetLastError());
}

void copy_rows_f32(const float* x, int ldx, float* y, int ldy, int rows, int cols,
                   hipStream_t stream) {
  if (rows <= 0) return;
  BARK_LAUNCH(copy_rows_kernel, dim3(ceil_div(cols, 256), rows), dim3(256), 0, stream, x,
                     ldx, y, ldy, cols);
  BARK_HIP_CHECK(hipGetLastError());
}

void sub_conv1_dw(const float* mel, int frames, const float* w1, const float* b1, int vlen1,
                  const float* wd, const float* bd, int vlen2, half* out, hipStream_t stream) {
  const int f1 = (frames - 1) / 2 + 1, t2 = (f1 - 1) / 2 + 1;
  static_assert(SUB_CH % FD_CH == 0, "channel chunks must tile the 256 channels");
  BARK_LAUNCH(conv1_dw_kernel, dim3(ceil_div(t2, FD_ROWS), SUB_CH / FD_CH), dim3(256), 0, stream, mel, frames,
              f1, vlen1, w1, b1, wd, bd, out, t2, vlen2);
  BARK_HIP_CHECK(hipGetLastError());
}

void sub_dwconv(const half* in, int t_in, int m_in, const float* w, const float* b, half* out,
                int vlen, hipStream_t stream) {
  const int t_out = (t_in - 1) / 2 + 1, m_out = (m_in - 1) / 2 + 1;
  BARK_LAUNCH(sub_dw_kernel, dim3(ceil_div(t_out * m_out, DW2_PIX)), dim3(256), 0,
                     stream, in, t_in, m_in, w, b, out, t_out, m_out, vlen);
  BARK_HIP_CHECK(hipGetLastError());
}

}  // namespace bark
