// GPU-resident greedy TDT decoding: the loop of TdtDecoder::decode_rayon
// (src/tdt.rs:374-414) with the decoder state, the frame pointer and the
// emitted tokens kept in device memory, as GpuTdtDecoder does
// (src/tdt_gpu.rs:1-7, 206-300).
//
// A decode step is five launches on one stream; each reads only what the
// launches before it wrote, so kernel boundaries are the only synchronisation,
// and the control state (frame, step count, parity of the h buffers, whether
// the LSTM runs) lives in device memory:
//   joint  x = relu(pooler[frame] + dec); scores of the 8198 head rows (8193
//          tokens + 5 durations, f16 weights, f32 sums, src/tdt.rs:217-288)
//          over G workgroups, each leaving its best token and best duration;
//   decide one wave reduces the partials and applies the step: blank: frame +=
//          max(dur, 1); token: record {id, frame, dur}, run the LSTM, frame +=
//          dur (src/tdt.rs:386-412); `done` once the loop would exit (frame >=
//          T or the step guard T * 14 + 64);
//   lstm   (twice) one wave per channel: its i, f, g, o gate rows of w_ih and
//          w_hh (8 row dots, 8 lanes each), gate = b_ih + b_hh + w_ih.x +
//          w_hh.h_old, c = f c + i g, h = o tanh(c) (src/tdt.rs:179-214);
//   proj   dec = b + W h1 (src/tdt.rs:515-529).
// Launches after `done`, and lstm / proj after a blank, return at once. The
// host queues steps in chunks and reads back only the state words. Row dots
// read each 1280-byte f16 row with 8 lanes (ten 16-byte loads each, issued
// before the input vector is staged in LDS, so both loads overlap).
//
// Measured alternatives: deciding in the joint's last workgroup (an arrival
// counter) and a single cooperative launch with grid barriers between the
// phases were both slower than these launch boundaries (arrivals of 256
// workgroups on one counter serialise; a cross-XCD barrier costs more than a
// dependent launch).
//
// The argmax order is total — higher score first, then the lower row — so the
// result does not depend on how rows are spread over workgroups and lanes and
// equals the reference's first-maximum scan. Dot products are f32 sums in a
// different order than the reference's 8-lane AVX blocks, so scores agree to
// rounding and greedy decisions agree unless two scores tie to within it.
#include "kernels.h"

namespace bark {
namespace {

constexpr int DH = 640, GS = 4 * DH;
constexpr int VOCAB = 8193, NROWS = VOCAB + 5, BLANK = 8192;
constexpr int WAVES = 8, THREADS = 64 * WAVES;
constexpr int GROUPS = THREADS / 8;  // 8-lane row groups per workgroup
constexpr int ROW_LOADS = DH / 8 / 8;  // 16-byte loads per lane per row (10)
constexpr int NONE = 0x7fffffff;

// state words (int32)
enum { S_FRAME, S_DONE, S_NTOK, S_GUARD, S_TOKEN, S_EMIT, S_PAR, S_LSTM, S_TLEN, S_MAXSTEPS, S_CAP, S_WORDS };
typedef _Float16 h2v __attribute__((ext_vector_type(2)));

__device__ inline float2 halves(uint32_t u) {
  const h2v h = __builtin_bit_cast(h2v, u);
  return make_float2((float)h.x, (float)h.y);
}

// A 640-entry f16 row as the 8 lanes of a group hold it (sub = lane & 7):
// 16-byte chunks sub, sub + 8, ..., sub + 72
struct Row {
  uint4 w[ROW_LOADS];
  __device__ void load(const half* row, int sub) {
    const uint4* r = reinterpret_cast<const uint4*>(row);
#pragma unroll
    for (int j = 0; j < ROW_LOADS; ++j) w[j] = r[sub + 8 * j];
  }
  // row . x (x: 640 f32 in LDS); every lane of the group returns the sum
  __device__ float dot(const float* xs, int sub) const {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < ROW_LOADS; ++j) {
      const float* x = xs + 8 * (sub + 8 * j);
      const float4 xa = *reinterpret_cast<const float4*>(x);
      const float4 xb = *reinterpret_cast<const float4*>(x + 4);
      const float2 a = halves(w[j].x), b = halves(w[j].y), c = halves(w[j].z), d = halves(w[j].w);
      s = fmaf(a.x, xa.x, s);
      s = fmaf(a.y, xa.y, s);
      s = fmaf(b.x, xa.z, s);
      s = fmaf(b.y, xa.w, s);
      s = fmaf(c.x, xb.x, s);
      s = fmaf(c.y, xb.y, s);
      s = fmaf(d.x, xb.z, s);
      s = fmaf(d.y, xb.w, s);
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    return s;
  }
};

// (score, row) order of the argmax: higher score, then lower row
__device__ inline bool better(float s, int i, float bs, int bi) { return s > bs || (s == bs && i < bi); }

struct Best {
  float ts, ds;
  int ti, di;
  __device__ void take(float s, int i, float t, int j) {
    if (better(s, i, ts, ti)) ts = s, ti = i;
    if (better(t, j, ds, di)) ds = t, di = j;
  }
  __device__ void wave_reduce(int from) {  // xor-butterfly over lanes `from`, 2*from, ... 32
    for (int o = from; o < 64; o <<= 1)
      take(__shfl_xor(ts, o, 64), __shfl_xor(ti, o, 64), __shfl_xor(ds, o, 64), __shfl_xor(di, o, 64));
  }
};

struct Lds {
  __attribute__((aligned(16))) float xs[DH];
  __attribute__((aligned(16))) float hs[DH];
  Best wave_best[WAVES];
  int tok, dur;
};

struct Weights {
  const float* embed;
  const half *w_ih, *w_hh, *proj_w, *head_w;
  const float *b_ih, *b_hh, *proj_b, *head_b;
};

// ---------------------------------------------------------------- phases --

// joint scores of rows wg, wg + G, ... ; the workgroup's best token and best
// duration go to part[wg]
__device__ void phase_joint(const Weights& W, const float* enc, const float* dec, float4* part, int G, int wg,
                            Lds& sh) {
  const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7;
  const int r = wg + G * grp;
  Row row;
  if (r < NROWS) row.load(W.head_w + (size_t)r * DH, sub);
  for (int k = threadIdx.x; k < DH; k += THREADS) sh.xs[k] = fmaxf(enc[k] + dec[k], 0.0f);
  __syncthreads();
  Best b{-INFINITY, -INFINITY, NONE, NONE};
  if (r < NROWS) {
    const float sc = W.head_b[r] + row.dot(sh.xs, sub);
    if (r < VOCAB)
      b.ts = sc, b.ti = r;
    else
      b.ds = sc, b.di = r;
  }
  b.wave_reduce(8);
  if ((threadIdx.x & 63) == 0) sh.wave_best[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < WAVES; ++i) {
      const Best& o = sh.wave_best[i];
      b.take(o.ts, o.ti, o.ds, o.di);
    }
    part[wg] = make_float4(b.ts, __int_as_float(b.ti), b.ds, __int_as_float(b.di));
  }
}

// reduce G partials (wave 0) -> sh.tok, sh.dur for the whole workgroup
__device__ void phase_decide(const float4* part, int G, Lds& sh) {
  if (threadIdx.x < 64) {
    Best b{-INFINITY, -INFINITY, NONE, NONE};
    for (int g = threadIdx.x; g < G; g += 64) {
      const float4 c = part[g];
      b.take(c.x, __float_as_int(c.y), c.z, __float_as_int(c.w));
    }
    b.wave_reduce(1);
    if (threadIdx.x == 0) {
      // with NaN everywhere no row qualifies: token 0 (the reference's initial
      // best) and duration 0 keep the control flow in range
      sh.tok = b.ti < VOCAB ? b.ti : 0;
      sh.dur = (b.di >= VOCAB && b.di < NROWS) ? b.di - VOCAB : 0;
    }
  }
  __syncthreads();
}

__device__ inline float sigmoid_ref(float x) { return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-x))); }

// one LSTM layer: input x, previous h (nullptr = zeros, and c = 0), new h into
// h_new; c of the layer updated in place. Channel ch is owned by wave ch / G of
// workgroup ch % G, the same owner every step.
__device__ void phase_lstm(const Weights& W, int layer, const float* x, const float* h_old, float* h_new, float* c,
                           int G, int wg, Lds& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ch = wg + G * wave;
  const int grp = lane >> 3, sub = lane & 7;
  const int kind = grp >> 1, hh = grp & 1;  // gate i, f, g, o; input or hidden weights
  Row row;
  if (ch < DH) row.load((hh ? W.w_hh : W.w_ih) + ((size_t)layer * GS + kind * DH + ch) * DH, sub);
  for (int k = threadIdx.x; k < DH; k += THREADS) {
    sh.xs[k] = x[k];
    sh.hs[k] = h_old ? h_old[k] : 0.0f;
  }
  __syncthreads();
  if (ch < DH) {
    const float v = row.dot(hh ? sh.hs : sh.xs, sub);
    float g4[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float di = __shfl(v, 16 * k, 64), dh = __shfl(v, 16 * k + 8, 64);
      const int rk = layer * GS + k * DH + ch;
      g4[k] = ((W.b_ih[rk] + W.b_hh[rk]) + di) + dh;
    }
    if (lane == 0) {
      const float ig = sigmoid_ref(g4[0]), fg = sigmoid_ref(g4[1]), gg = tanhf(g4[2]);
      const float c_old = h_old ? c[ch] : 0.0f;
      const float cn = __fadd_rn(__fmul_rn(fg, c_old), __fmul_rn(ig, gg));
      c[ch] = cn;
      h_new[ch] = __fmul_rn(sigmoid_ref(g4[3]), tanhf(cn));
    }
  }
}

// dec rows wg, wg + G, ... = b + W h1
__device__ void phase_proj(const Weights& W, const float* h1, float* dec, int G, int wg, Lds& sh) {
  const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7;
  const int r = wg + G * grp;
  Row row;
  if (r < DH) row.load(W.proj_w + (size_t)r * DH, sub);
  for (int k = threadIdx.x; k < DH; k += THREADS) sh.xs[k] = h1[k];
  __syncthreads();
  if (r < DH) {
    const float d = row.dot(sh.xs, sub);
    if (sub == 0) dec[r] = W.proj_b[r] + d;
  }
}

// --------------------------------------------------------- stepped driver --

__global__ void __launch_bounds__(THREADS) tdt_joint_kernel(Weights W, const float* pooler, const float* dec,
                                                            const int* state, float4* part) {
  if (state[S_DONE]) return;
  __shared__ Lds sh;
  phase_joint(W, pooler + (size_t)state[S_FRAME] * DH, dec, part, gridDim.x, blockIdx.x, sh);
}

// the step's decision: one wave reduces the joint partials and applies it
__global__ void __launch_bounds__(64) tdt_decide_kernel(int* state, const float4* part, int G, uint32_t* tokens) {
  if (state[S_DONE]) return;
  __shared__ Lds sh;
  phase_decide(part, G, sh);
  if (threadIdx.x != 0) return;
  const int tok = sh.tok, dur = sh.dur;
  int frame = state[S_FRAME];
  const int guard = state[S_GUARD] + 1;
  state[S_GUARD] = guard;
  int emit = 0;
  if (tok == BLANK) {
    frame += max(dur, 1);
  } else {
    const int n = state[S_NTOK];
    if (n < state[S_CAP]) {
      tokens[3 * n] = (uint32_t)tok;
      tokens[3 * n + 1] = (uint32_t)frame;
      tokens[3 * n + 2] = (uint32_t)dur;
    }
    state[S_NTOK] = n + 1;
    frame += dur;
    emit = 1;
  }
  const int done = frame >= state[S_TLEN] || guard >= state[S_MAXSTEPS];
  state[S_FRAME] = frame;
  state[S_DONE] = done;
  // the new decoder state is only needed if another step follows
  state[S_EMIT] = emit && !done;
  if (emit && !done) {
    state[S_TOKEN] = tok;
    state[S_PAR] = state[S_LSTM] & 1;
    state[S_LSTM] += 1;
  }
}

// h[layer][S_PAR] holds the old state, h[layer][S_PAR ^ 1] receives the new one
__global__ void __launch_bounds__(THREADS) tdt_lstm_kernel(Weights W, int layer, const int* state, float* h,
                                                           float* c) {
  if (!state[S_EMIT]) return;
  __shared__ Lds sh;
  const int p = state[S_PAR];
  const bool first = state[S_LSTM] == 1;  // the start step: h = c = 0
  const float* x = layer == 0 ? W.embed + (size_t)state[S_TOKEN] * DH : h + (size_t)(p ^ 1) * DH;
  phase_lstm(W, layer, x, first ? nullptr : h + (size_t)(layer * 2 + p) * DH, h + (size_t)(layer * 2 + (p ^ 1)) * DH,
             c + (size_t)layer * DH, gridDim.x, blockIdx.x, sh);
}

__global__ void __launch_bounds__(THREADS) tdt_proj_kernel(Weights W, const int* state, const float* h,
                                                           float* dec) {
  if (!state[S_EMIT]) return;
  __shared__ Lds sh;
  phase_proj(W, h + (size_t)(2 + (state[S_PAR] ^ 1)) * DH, dec, gridDim.x, blockIdx.x, sh);
}

__global__ void tdt_init_kernel(int* state, int t_len, int max_steps, int cap) {
  if (threadIdx.x == 0) {
    state[S_FRAME] = 0;
    state[S_DONE] = t_len <= 0;
    state[S_NTOK] = 0;
    state[S_GUARD] = 0;
    state[S_TOKEN] = BLANK;
    state[S_EMIT] = 1;
    state[S_PAR] = 0;
    state[S_LSTM] = 1;
    state[S_TLEN] = t_len;
    state[S_MAXSTEPS] = max_steps;
    state[S_CAP] = cap;
  }
}

Weights weights_of(const TdtDev& d) {
  return Weights{d.embed, d.w_ih, d.w_hh, d.proj_w, d.head_w, d.b_ih, d.b_hh, d.proj_b, d.head_b};
}

constexpr int STEP_G = TDT_PARTIALS;  // workgroups per phase

}  // namespace

int tdt_state_words() { return S_WORDS; }
int tdt_frame_word() { return S_FRAME; }
int tdt_done_word() { return S_DONE; }
int tdt_count_word() { return S_NTOK; }
int tdt_max_steps(int t_len) { return t_len * (10 + 4) + 64; }  // src/tdt.rs:381 (MAX_SYMBOLS = 10)

void tdt_begin(const TdtDev& d, int t_len, int cap, hipStream_t st) {
  const Weights W = weights_of(d);
  BARK_LAUNCH(tdt_init_kernel, dim3(1), dim3(64), 0, st, d.state, t_len, tdt_max_steps(t_len), cap);
  for (int layer = 0; layer < 2; ++layer)
    BARK_LAUNCH(tdt_lstm_kernel, dim3(STEP_G), dim3(THREADS), 0, st, W, layer, (const int*)d.state, d.h, d.c);
  BARK_LAUNCH(tdt_proj_kernel, dim3(STEP_G), dim3(THREADS), 0, st, W, (const int*)d.state, (const float*)d.h, d.dec);
  BARK_HIP_CHECK(hipGetLastError());
}

void tdt_steps(const TdtDev& d, const float* pooler, int steps, hipStream_t st) {
  const Weights W = weights_of(d);
  float4* part = reinterpret_cast<float4*>(d.partials);
  for (int s = 0; s < steps; ++s) {
    BARK_LAUNCH(tdt_joint_kernel, dim3(STEP_G), dim3(THREADS), 0, st, W, pooler, (const float*)d.dec,
                (const int*)d.state, part);
    BARK_LAUNCH(tdt_decide_kernel, dim3(1), dim3(64), 0, st, d.state, (const float4*)part, STEP_G, d.tokens);
    for (int layer = 0; layer < 2; ++layer)
      BARK_LAUNCH(tdt_lstm_kernel, dim3(STEP_G), dim3(THREADS), 0, st, W, layer, (const int*)d.state, d.h, d.c);
    BARK_LAUNCH(tdt_proj_kernel, dim3(STEP_G), dim3(THREADS), 0, st, W, (const int*)d.state, (const float*)d.h,
                d.dec);
  }
  BARK_HIP_CHECK(hipGetLastError());
}

}  // namespace bark
