// Log-mel front end on the GPU: MelFrontend::compute (src/mel.rs:41-140).
//
// wave (16 kHz mono f32) -> preemphasis 0.97 -> 512-sample frames every 160
// samples, centre-padded with zeros, times the symmetric 400-point Hann
// window -> |FFT|^2 of bins 0..256 -> 128 slaney mel sums -> ln(s + 2^-24)
// -> per-bin mean / sample std over the valid frames -> (x - mean) /
// (std + 1e-5), padded frames zero. Products and sums the reference rounds
// one operation at a time (preemphasis, power, mel sums) are rounded the same
// way here (no fused multiply-adds). The FFT is radix-2 in f64 and its power
// is rounded to f32: the reference's f32 rustfft is itself a few f32 ulps off
// the exact spectrum, and an f32 radix-2 FFT here was ~10x further off (1e-3 on
// the normalised features of weak bins against an f64 pipeline). The
// statistics accumulate in f64.
#include "kernels.h"

namespace bark {
namespace {

constexpr int HOP = 160;
constexpr int NFFT = 512;
constexpr int NBIN = NFFT / 2 + 1;  // 257
constexpr int NMEL = MEL;           // 128
constexpr int FRAMES_PER_WG = 4;    // one wave per frame
constexpr int STAT_CHUNK = 64;      // frames per partial-sum chunk

__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline int bitrev9(int i) { return (int)(__builtin_bitreverse32((uint32_t)i) >> 23); }

// One frame per wave: windowed samples in bit-reversed order, nine radix-2
// stages through LDS, the power of bins 0..256, then lane l sums mel rows l
// and l + 64 over their nonzero filter entries in ascending bin order.
__global__ void __launch_bounds__(256) mel_frame_kernel(const float* wave, long n, int n_frames,
                                                        const float* window, const double* twid,
                                                        const int* rows, const float* vals, float* raw) {
  __shared__ double re[FRAMES_PER_WG][NFFT], im[FRAMES_PER_WG][NFFT];
  __shared__ float pw[FRAMES_PER_WG][NBIN];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * FRAMES_PER_WG + w;
  if (t >= n_frames) return;  // whole wave
  double* xr = re[w];
  double* xi = im[w];
  float* xp = pw[w];
  const long s0 = (long)t * HOP - NFFT / 2;
#pragma unroll
  for (int j = 0; j < NFFT / 64; ++j) {
    const int i = lane + 64 * j;
    const long s = s0 + i;
    float v = 0.0f;
    if (s >= 0 && s < n) v = s == 0 ? wave[0] : __fsub_rn(wave[s], __fmul_rn(0.97f, wave[s - 1]));
    const int r = bitrev9(i);
    xr[r] = (double)__fmul_rn(v, window[i]);
    xi[r] = 0.0;
  }
  wave_sync();
  for (int h = 1; h < NFFT; h <<= 1) {  // butterflies of span 2h
    const int tstep = NFFT / (2 * h);
#pragma unroll
    for (int j = 0; j < NFFT / 2 / 64; ++j) {
      const int b = lane + 64 * j;
      const int pos = b & (h - 1);
      const int i0 = ((b - pos) << 1) + pos, i1 = i0 + h;
      const double c = twid[pos * tstep], sn = twid[NFFT / 2 + pos * tstep];  // e^{-2 pi i pos / 2h}
      const double ar = xr[i1], ai = xi[i1];
      const double vr = ar * c + ai * sn, vi = ai * c - ar * sn;
      const double ur = xr[i0], ui = xi[i0];
      xr[i0] = ur + vr;
      xi[i0] = ui + vi;
      xr[i1] = ur - vr;
      xi[i1] = ui - vi;
    }
    wave_sync();
  }
  // power of bins 0..256, rounded to f32
  for (int k = lane; k < NBIN; k += 64) xp[k] = (float)(xr[k] * xr[k] + xi[k] * xi[k]);
  wave_sync();
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int m = lane + 64 * q;
    const int first = rows[3 * m], count = rows[3 * m + 1], off = rows[3 * m + 2];
    float s = 0.0f;
    for (int e = 0; e < count; ++e) s = __fadd_rn(s, __fmul_rn(vals[off + e], xp[first + e]));
    raw[(size_t)t * NMEL + m] = logf(s + 5.9604644775390625e-8f);  // 2^-24
  }
}

// Partial sums over a chunk of valid frames: thread m of chunk c writes
// (sum x, sum x^2) of bin m in f64.
__global__ void __launch_bounds__(NMEL) mel_partial_kernel(const float* raw, int n_valid, double* part) {
  const int c = blockIdx.x, m = threadIdx.x;
  double s1 = 0.0, s2 = 0.0;
  const int t1 = min(n_valid, (c + 1) * STAT_CHUNK);
  for (int t = c * STAT_CHUNK; t < t1; ++t) {
    const double x = raw[(size_t)t * NMEL + m];
    s1 += x;
    s2 += x * x;
  }
  part[(size_t)c * 2 * NMEL + m] = s1;
  part[(size_t)c * 2 * NMEL + NMEL + m] = s2;
}

// mean and sample std (N - 1, at least 1) per bin from the chunk partials, in chunk order
__global__ void __launch_bounds__(NMEL) mel_stats_kernel(const double* part, int chunks, int n_valid,
                                                         float* stats) {
  const int m = threadIdx.x;
  double s1 = 0.0, s2 = 0.0;
  for (int c = 0; c < chunks; ++c) {
    s1 += part[(size_t)c * 2 * NMEL + m];
    s2 += part[(size_t)c * 2 * NMEL + NMEL + m];
  }
  const double nv = (double)max(n_valid, 1);
  const double mean = s1 / nv;
  const double var = fmax(s2 - nv * mean * mean, 0.0) / (double)max(n_valid - 1, 1);
  stats[m] = (float)mean;
  stats[NMEL + m] = (float)sqrt(var);
}

__global__ void __launch_bounds__(256) mel_norm_kernel(const float* raw, const float* stats, int n_frames,
                                                       int n_valid, float* out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)n_frames * NMEL) return;
  const int t = (int)(i / NMEL), m = (int)(i % NMEL);
  out[i] = t < n_valid ? __fdiv_rn(__fsub_rn(raw[i], stats[m]), __fadd_rn(stats[NMEL + m], 1e-5f)) : 0.0f;
}

}  // namespace

int mel_frames(long n_samples) { return (int)(1 + n_samples / HOP); }

size_t mel_workspace_bytes(long n_samples) {
  const int nf = mel_frames(n_samples);
  const int chunks = (nf + STAT_CHUNK - 1) / STAT_CHUNK;
  return (size_t)nf * NMEL * 4 + (size_t)chunks * 2 * NMEL * 8 + 2 * NMEL * 4 + 256;
}

void mel_features(const float* wave, long n_samples, const MelTables& tb, void* workspace, float* out,
                  hipStream_t st) {
  BARK_REQUIRE(n_samples > 0 && n_samples < (1l << 40), "mel: bad sample count");
  BARK_REQUIRE(tb.window && tb.twiddle && tb.rows && tb.vals, "mel: filterbank not set");
  const int nf = mel_frames(n_samples), nv = (int)(n_samples / HOP);
  const int chunks = (std::max(nv, 1) + STAT_CHUNK - 1) / STAT_CHUNK;
  char* ws = static_cast<char*>(workspace);
  float* raw = reinterpret_cast<float*>(ws);
  double* part = reinterpret_cast<double*>(ws + (((size_t)nf * NMEL * 4 + 255) & ~(size_t)255));
  float* stats = reinterpret_cast<float*>(reinterpret_cast<char*>(part) + (size_t)chunks * 2 * NMEL * 8);
  BARK_LAUNCH(mel_frame_kernel, dim3((nf + FRAMES_PER_WG - 1) / FRAMES_PER_WG), dim3(256), 0, st, wave,
              n_samples, nf, tb.window, tb.twiddle, tb.rows, tb.vals, raw);
  BARK_HIP_CHECK(hipGetLastError());
  BARK_LAUNCH(mel_partial_kernel, dim3(chunks), dim3(NMEL), 0, st, raw, nv, part);
  BARK_HIP_CHECK(hipGetLastError());
  BARK_LAUNCH(mel_stats_kernel, dim3(1), dim3(NMEL), 0, st, part, chunks, nv, stats);
  BARK_HIP_CHECK(hipGetLastError());
  BARK_LAUNCH(mel_norm_kernel, dim3((unsigned)(((size_t)nf * NMEL + 255) / 256)), dim3(256), 0, st, raw, stats,
              nf, nv, out);
  BARK_HIP_CHECK(hipGetLastError());
}

}  // namespace bark
