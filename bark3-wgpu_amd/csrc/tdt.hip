// GPU-resident greedy TDT decoding: the loop of TdtDecoder::decode_rayon
// (src/tdt.rs:374-414) with the decoder state, the frame pointer and the
// emitted tokens kept in device memory, as GpuTdtDecoder does
// (src/tdt_gpu.rs:1-7, 206-300).
//
// The decode is a chain of launches of one kernel on one stream; each launch
// runs the phase its control state (in device memory) names and leaves the
// next control state, so kernel boundaries are the only synchronisation:
//   joint  x = relu(pooler[frame] + dec); scores of the 8198 head rows (8193
//          tokens + 5 durations, f16 weights, f32 sums, src/tdt.rs:217-288)
//          over G workgroups, each leaving its best token and best duration;
//   decide every workgroup reduces the partials to the step's decision (the
//          same everywhere): blank: frame += max(dur, 1) (src/tdt.rs:386-412),
//          and the next step's joint runs in the same launch (dec is
//          unchanged); token: record {id, frame, dur}, frame += dur, and LSTM
//          layer 0 on its embedding in the same launch: one wave per channel
//          holds its i, f, g, o gate rows of w_ih and w_hh (8 row dots, 8 lanes
//          each), gate = b_ih + b_hh + w_ih.x + w_hh.h_old, c = f c + i g,
//          h = o tanh(c) (src/tdt.rs:179-214); `done` once the loop would exit
//          (frame >= T or the step guard T * 14 + 64);
//   lstm1  layer 1 on the new h0;
//   proj   dec = b + W h1 (src/tdt.rs:515-529).
// A blank step costs one launch, a token step four (decide, lstm1, proj,
// joint). The host queues launches in chunks and reads back only the control
// state. Row dots read each 1280-byte f16 row with 8 lanes (ten 16-byte loads
// each, issued before the input vector is staged in LDS or the decision is
// known, so the loads overlap).
//
// Measured alternatives (T = 2207, 1267 steps): one launch per phase with a
// separate one-wave decision, 24.4 ms; the decision folded into the layer-0
// launch (four launches every step), 19-21 ms; this phase chain, 16 ms. The
// decision in the joint's last workgroup via an arrival counter (256 arrivals
// on one counter serialise) and a single cooperative launch with grid
// barriers between the phases (a cross-XCD barrier costs more than a dependent
// launch) were both slower.
//
// The argmax order is total — higher score first, then the lower row — so the
// result does not depend on how rows are spread over workgroups and lanes and
// equals the reference's first-maximum scan. Dot products are f32 sums in a
// different order than the reference's 8-lane AVX blocks, so scores agree to
// rounding and greedy decisions agree unless two scores tie to within it.
#include <cstdio>
#include <cstdlib>

#include "kernels.h"

namespace bark {
namespace {

constexpr int DH = 640, GS = 4 * DH;
constexpr int VOCAB = 8193, NROWS = VOCAB + 5, BLANK = 8192;
constexpr int WAVES = 8, THREADS = 64 * WAVES;
constexpr int ROW_LOADS = DH / 8 / 8;  // 16-byte loads per lane per row (10)
constexpr int NONE = 0x7fffffff;

// state words (int32)
enum { S_PHASE, S_FRAME, S_DONE, S_NTOK, S_GUARD, S_PAR, S_LSTM, S_PQ, S_TLEN, S_MAXSTEPS, S_CAP, S_ROW0, S_TOK0,
       S_WORDS };
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

// the head row of this lane group in the joint: rows wg, wg + G, ...
__device__ inline bool joint_row(const Weights& W, int G, int wg, Row& row) {
  const int r = wg + G * (threadIdx.x >> 3);
  if (r >= NROWS) return false;
  row.load(W.head_w + (size_t)r * DH, threadIdx.x & 7);
  return true;
}

// joint scores of rows wg, wg + G, ... (rows loaded by joint_row); the
// workgroup's best token and best duration go to part[wg]
__device__ void phase_joint(const Weights& W, const Row& row, bool has_row, const float* enc, const float* dec,
                            float4* part, int G, int wg, Lds& sh) {
  for (int k = threadIdx.x; k < DH; k += THREADS) sh.xs[k] = fmaxf(enc[k] + dec[k], 0.0f);
  __syncthreads();
  Best b{-INFINITY, -INFINITY, NONE, NONE};
  if (has_row) {
    const int r = wg + G * (threadIdx.x >> 3);
    const float sc = W.head_b[r] + row.dot(sh.xs, threadIdx.x & 7);
    // a row competes only with a score above -inf (NaN never does), as the
    // reference's `score > best` scan from -inf
    if (sc > -INFINITY) {
      if (r < VOCAB)
        b.ts = sc, b.ti = r;
      else
        b.ds = sc, b.di = r;
    }
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
      // no qualifying row: token 0 and duration row 0, i.e. 0 - 8193 (the
      // reference's initial best; its u32 duration wraps and ends the decode)
      sh.tok = b.ti < VOCAB ? b.ti : 0;
      sh.dur = (b.di >= VOCAB && b.di < NROWS) ? b.di - VOCAB : -VOCAB;
    }
  }
  __syncthreads();
}

__device__ inline float sigmoid_ref(float x) { return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-x))); }

// one LSTM layer: input x, previous h (nullptr = zeros, and c = 0), new h into
// h_new; c of the layer updated in place. Channel ch is owned by wave ch / G of
// workgroup ch % G, the same owner every step; lane group g of the wave holds
// gate row g / 2 (i, f, g, o) of w_ih (g even) or w_hh (g odd), loaded by
// lstm_row before the input is known.
__device__ inline bool lstm_row(const Weights& W, int layer, int G, int wg, Row& row) {
  const int lane = threadIdx.x & 63, ch = wg + G * (threadIdx.x >> 6);
  if (ch >= DH) return false;
  const int grp = lane >> 3;
  row.load(((grp & 1) ? W.w_hh : W.w_ih) + ((size_t)layer * GS + (grp >> 1) * DH + ch) * DH, lane & 7);
  return true;
}

__device__ void phase_lstm(const Weights& W, int layer, const Row& row, bool has_row, const float* x,
                           const float* h_old, float* h_new, float* c, int G, int wg, Lds& sh) {
  for (int k = threadIdx.x; k < DH; k += THREADS) {
    sh.xs[k] = x[k];
    sh.hs[k] = h_old ? h_old[k] : 0.0f;
  }
  __syncthreads();
  if (!has_row) return;
  const int lane = threadIdx.x & 63, ch = wg + G * (threadIdx.x >> 6);
  const float v = row.dot(((lane >> 3) & 1) ? sh.hs : sh.xs, lane & 7);
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

// ---------------------------------------------------------- the launches --

// Every launch runs the phase the control state names and leaves the next
// control state in `out` (written by workgroup 0; `in` stays as it was, so
// every workgroup reads the same values). Every workgroup reduces the joint
// partials itself, so the decision needs no launch of its own:
//   START   LSTM layer 0 on the blank embedding from h = c = 0   -> L1
//   L1      LSTM layer 1 on the new h0                           -> PROJ
//   PROJ    dec = b + W h1                                       -> JOINT
//   JOINT   joint partials at `frame` into set q                 -> DECIDE
//   DECIDE  decision from set q (src/tdt.rs:386-412):
//             done (frame >= T or the step guard)                -> DONE
//             blank: frame += max(dur, 1), joint partials at the
//             new frame into set q ^ 1                           -> DECIDE
//             token: record {id, frame, dur}, frame += dur,
//             LSTM layer 0 on its embedding                      -> L1
//   DONE    nothing
// A run of blanks costs one launch per step; a token step four.
enum { PH_START, PH_L1, PH_PROJ, PH_JOINT, PH_DECIDE, PH_DONE };

__host__ __device__ inline int tdt_max_steps_of(int t_len) { return t_len * (10 + 4) + 64; }  // src/tdt.rs:381


// Utterance b = blockIdx.y of a batch: its control state, h, c, dec, partials
// and token records live at fixed strides; its pooler rows start at row
// S_ROW0 of `pooler` and its token records at record S_TOK0.
__global__ void __launch_bounds__(THREADS) tdt_advance_kernel(Weights W, const float* pooler, const int* in_all,
                                                              int* out_all, float4* part_all, uint32_t* tokens,
                                                              float* h_all, float* c_all, float* dec_all) {
  __shared__ Lds sh;
  const int G = gridDim.x, wg = blockIdx.x, u = blockIdx.y;
  const int* in = in_all + (size_t)u * 2 * S_WORDS;
  int* out = out_all + (size_t)u * 2 * S_WORDS;
  float4* part = part_all + (size_t)u * 2 * TDT_PARTIALS;
  float* h = h_all + (size_t)u * 4 * DH;
  float* c = c_all + (size_t)u * 2 * DH;
  float* dec = dec_all + (size_t)u * DH;
  if (in[S_PHASE] == PH_DONE) {  // keep the state current in both buffers
    if (wg == 0 && threadIdx.x < S_WORDS) out[threadIdx.x] = in[threadIdx.x];
    return;
  }
  pooler += (size_t)in[S_ROW0] * DH;
  tokens += (size_t)in[S_TOK0] * 3;
  const int phase = in[S_PHASE];
  // the control state this launch leaves (workgroup 0 writes it at the end)
  int frame = in[S_FRAME], ntok = in[S_NTOK], guard = in[S_GUARD], lstm = in[S_LSTM], par = in[S_PAR];
  int q = in[S_PQ], next = phase, done = in[S_DONE];
  Row row;
  bool has_row;
  switch (phase) {
    case PH_START:  // h[0][1] = lstm0(embed[blank]; h = c = 0)
      has_row = lstm_row(W, 0, G, wg, row);
      phase_lstm(W, 0, row, has_row, W.embed + (size_t)BLANK * DH, nullptr, h + DH, c, G, wg, sh);
      next = PH_L1;
      break;
    case PH_L1: {  // h[1][par ^ 1] = lstm1(h[0][par ^ 1]; h[1][par])
      has_row = lstm_row(W, 1, G, wg, row);
      const bool first = lstm == 1;
      phase_lstm(W, 1, row, has_row, h + (size_t)(par ^ 1) * DH, first ? nullptr : h + (size_t)(2 + par) * DH,
                 h + (size_t)(2 + (par ^ 1)) * DH, c + DH, G, wg, sh);
      next = PH_PROJ;
      break;
    }
    case PH_PROJ:
      phase_proj(W, h + (size_t)(2 + (par ^ 1)) * DH, dec, G, wg, sh);
      next = PH_JOINT;
      break;
    case PH_JOINT:
      has_row = joint_row(W, G, wg, row);
      phase_joint(W, row, has_row, pooler + (size_t)frame * DH, dec, part + q * TDT_PARTIALS, G, wg, sh);
      next = PH_DECIDE;
      break;
    case PH_DECIDE: {
      has_row = joint_row(W, G, wg, row);  // the next joint's rows, in case this step is a blank
      phase_decide(part + q * TDT_PARTIALS, G, sh);
      const int tok = sh.tok, dur = sh.dur;
      ++guard;
      if (dur < 0) {  // a wrapped duration moves the frame past any T
        if (tok != BLANK && wg == 0 && threadIdx.x == 0 && ntok < in[S_CAP]) {
          tokens[3 * ntok] = (uint32_t)tok;
          tokens[3 * ntok + 1] = (uint32_t)frame;
          tokens[3 * ntok + 2] = (uint32_t)dur;
        }
        ntok += tok != BLANK;
        frame = in[S_TLEN];
      } else if (tok == BLANK) {
        frame += max(dur, 1);
      } else {
        if (wg == 0 && threadIdx.x == 0 && ntok < in[S_CAP]) {
          tokens[3 * ntok] = (uint32_t)tok;
          tokens[3 * ntok + 1] = (uint32_t)frame;
          tokens[3 * ntok + 2] = (uint32_t)dur;
        }
        ++ntok;
        frame += dur;
      }
      done = frame >= in[S_TLEN] || guard >= in[S_MAXSTEPS];
      if (done) {
        next = PH_DONE;
      } else if (tok == BLANK) {  // dec is unchanged: the next step's joint right away
        q ^= 1;
        phase_joint(W, row, has_row, pooler + (size_t)frame * DH, dec, part + q * TDT_PARTIALS, G, wg, sh);
      } else {
        par = lstm & 1;
        ++lstm;
        has_row = lstm_row(W, 0, G, wg, row);
        phase_lstm(W, 0, row, has_row, W.embed + (size_t)tok * DH, h + (size_t)par * DH, h + (size_t)(par ^ 1) * DH,
                   c, G, wg, sh);
        next = PH_L1;
      }
      break;
    }
    default:
      break;
  }
  if (wg == 0 && threadIdx.x < S_WORDS) {
    int v = in[threadIdx.x];
    switch (threadIdx.x) {
      case S_PHASE: v = next; break;
      case S_FRAME: v = frame; break;
      case S_DONE: v = done; break;
      case S_NTOK: v = ntok; break;
      case S_GUARD: v = guard; break;
      case S_PAR: v = par; break;
      case S_LSTM: v = lstm; break;
      case S_PQ: v = q; break;
      default: break;
    }
    out[threadIdx.x] = v;
  }
}

// per utterance: {t_len, pooler row, first token record, record capacity}
__global__ void tdt_init_kernel(int* state_all, const int* params, int batch) {
  const int u = blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= batch) return;
  int* state = state_all + (size_t)u * 2 * S_WORDS;  // the first buffer of the pair
  const int t_len = params[4 * u];
  state[S_PHASE] = t_len > 0 ? PH_START : PH_DONE;
  state[S_FRAME] = 0;
  state[S_DONE] = t_len <= 0;
  state[S_NTOK] = 0;
  state[S_GUARD] = 0;
  state[S_PAR] = 0;
  state[S_LSTM] = 1;
  state[S_PQ] = 0;
  state[S_TLEN] = t_len;
  state[S_MAXSTEPS] = tdt_max_steps_of(t_len);
  state[S_CAP] = params[4 * u + 3];
  state[S_ROW0] = params[4 * u + 1];
  state[S_TOK0] = params[4 * u + 2];
}

Weights weights_of(const TdtDev& d) {
  return Weights{d.embed, d.w_ih, d.w_hh, d.proj_w, d.head_w, d.b_ih, d.b_hh, d.proj_b, d.head_b};
}

// Workgroups per utterance and launch: every head row needs a row group (64
// per workgroup), every channel a wave (8 per workgroup), so at least 129.
// 160 measured best (one utterance: 129-256 within noise; a batch of 8 at
// T = 2207: 43 ms with 160, 57 ms with 129, 60 ms with 256).
// BARK_HIP_TDT_GROUPS overrides it for tuning.
int groups() {
  static const int g = [] {
    if (const char* e = std::getenv("BARK_HIP_TDT_GROUPS")) {
      const int v = std::atoi(e);
      if (v * 64 >= NROWS && v * WAVES >= DH && v <= TDT_PARTIALS) return v;
    }
    return 160;
  }();
  return g;
}

}  // namespace

int tdt_state_words() { return S_WORDS; }
int tdt_frame_word() { return S_FRAME; }
int tdt_done_word() { return S_DONE; }
int tdt_count_word() { return S_NTOK; }
int tdt_max_steps(int t_len) { return tdt_max_steps_of(t_len); }  // MAX_SYMBOLS = 10
long tdt_max_launches(int t_len) { return 4L * tdt_max_steps(t_len) + 4; }

void tdt_begin(const TdtDev& d, const int* d_params, int batch, hipStream_t st) {
  BARK_LAUNCH(tdt_init_kernel, dim3((batch + 63) / 64), dim3(64), 0, st, d.state, d_params, batch);
  BARK_HIP_CHECK(hipGetLastError());
}

const int* tdt_current(const TdtDev& d, long launches, int u) {
  return d.state + (size_t)u * 2 * S_WORDS + (launches & 1) * S_WORDS;
}

void tdt_launches(const TdtDev& d, const float* pooler, int batch, int n, long& launches, hipStream_t st) {
  const Weights W = weights_of(d);
  const int G = groups();
  float4* part = reinterpret_cast<float4*>(d.partials);
  for (int i = 0; i < n; ++i, ++launches) {
    const int* in = d.state + (launches & 1) * S_WORDS;
    int* out = d.state + ((launches + 1) & 1) * S_WORDS;
    BARK_LAUNCH(tdt_advance_kernel, dim3(G, batch), dim3(THREADS), 0, st, W, pooler, in, out, part, d.tokens, d.h,
                d.c, d.dec);
  }
  BARK_HIP_CHECK(hipGetLastError());
}

}  // namespace bark
