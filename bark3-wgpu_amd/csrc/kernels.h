// Host-side launchers for the gfx950 kernels (implemented in gemm.hip,
// attention.hip, ops.hip). All take device pointers and a stream, validate the
// shapes the kernels assume, and throw bark::Error on a mismatch.
#pragma once

#include <vector>

#include "common.h"

namespace bark {

// ---------------------------------------------------------------- GEMM --
// C[m, n] = sum_k A[m, k] * W[n, k]  (A f16 row-major, W f16 row-major or
// 4-bit codes + per-row 16-entry f16 table), f32 accumulation on MFMA, and an
// epilogue that consumes the f32 tile.
enum class Epi : int {
  StoreF32 = 0,      // out_f32[r][c] = v (+ bias[c])
  StoreF16 = 1,      // out_f16[r][c] = f16(v (+ bias[c]))
  Silu = 2,          // out_f16[r][c] = f16(silu(v))
  Resid = 3,         // out_f32[r][c] += scale * v
  Glu = 4,           // out_f32[r][c/2 pair] = a * sigmoid(b) (rows of W interleaved)
  Qkv = 5,           // head packing of scale*(q+bias_u), scale*(q+bias_v), k, v^T (f16)
  RelK = 6,          // rk[h][r][d] = f16(v)
  BiasReluF16 = 7,   // out_f16[r][c] = f16(max(v + bias[c], 0))
  FlattenReluF16 = 8, // pixel r = (t, m): out_f16[t][c*16+m] = f16(max(v+bias[c],0))
  StoreBF16 = 9,      // out (bf16 bits in out_f16)[r][c] = bf16(v (+ bias[c]))
  ResidHalf = 10      // out_f32[r][c] += 0.5 * v (the FFN half-step residual)
};

struct GemmWeight {
  // exactly one of (w16) or (codes, lut) is set
  const half* w16 = nullptr;     // (n, k) f16
  const uint8_t* codes = nullptr;  // (n, k/2) bytes, low nibble = even k
  const half* lut = nullptr;     // (n, 16) f16
  bool swizzled = false;  // codes in the swizzled nibble order (see gemm.hip)
  int n = 0, k = 0;
  bool lut4() const { return codes != nullptr; }
};

struct EpiArgs {
  float* out_f32 = nullptr;
  half* out_f16 = nullptr;
  int ldo = 0;
  const float* bias = nullptr;
  float scale = 1.0f;
  // Qkv
  half *qu = nullptr, *qv = nullptr, *kh = nullptr, *vt = nullptr;
  const float *bu = nullptr, *bv = nullptr;
  int mp = 0;  // rows of the head-major buffers
  // RelK
  half* rk = nullptr;
  int pp = 0;  // rows of rk per head
};

// Reorders 4-bit codes (rows x k/2 bytes, plain layout) into the swizzled
// layout the GEMM expands with fewer permutes. Host-side, in place.
void swizzle_codes(uint8_t* codes, size_t nbytes);

// Rows >= M of A read as zero and are not stored. a_bf16: A holds bf16 bits
// (converted to f16 while staging; exact for |a| in the f16 normal range).
void gemm(const half* A, int lda, int M, const GemmWeight& W, Epi epi, const EpiArgs& ea,
          hipStream_t stream, bool a_bf16 = false);

// Split-K GEMM into partial sums: K is cut into `splits` chunks of whole
// 256-k units (the first K/256 % splits chunks one unit longer) and chunk s
// writes its f32 product to
// part + s * M * ldo (row stride ldo). The consumer adds the chunks in order
// s = 0, 1, ... (see ResidIn), so the result depends on (N, K, splits) only,
// never on M or on which workgroup finished first.
void gemm_split(const half* A, int lda, int M, const GemmWeight& W, int splits, float* part,
                int ldo, hipStream_t stream, bool a_bf16 = false);
// The isolated linear C (M x N, dense) = A (M x K, lda = K) . W^T with output
// kind 0 = f32, 1 = f16, 2 = bf16; splits K over a workspace when M is small
// (grow-only, per stream, allocated on first need).
void gemm_isolated(const half* A, int M, const GemmWeight& W, void* C, int c_kind, hipStream_t stream,
                   bool a_bf16);
// The same kernels and results without any allocation: the partial sums live
// in a fixed device array of ISOLATED_SCRATCH_BYTES per GPU (shared by every
// call on that GPU: calls that overlap on one GPU race); larger splits are
// rejected.
constexpr size_t ISOLATED_SCRATCH_BYTES = (size_t)24 << 20;
void gemm_isolated_noalloc(const half* A, int M, const GemmWeight& W, void* C, int c_kind, hipStream_t stream,
                           bool a_bf16);
// Split-K count for the residual linears, a function of (N, K) only.
int residual_splits(int n, int k);

// Deferred residual update read by the LayerNorm kernels: x += scale * (p_0 +
// p_1 + ... ) with p_s = part + s * stride, summed in that order.
struct ResidIn {
  const float* part = nullptr;
  int splits = 0;  // 0: no pending update
  size_t stride = 0;
  float scale = 1.0f;
};

// ----------------------------------------------------------- attention --
// Work is cut into segments {row of the sequence's first frame, sequence
// length, first query of the 128-query tile (local), first key tile | (end key
// tile << 16)} with 64-key tiles. Workgroup lane l (one per head) runs segments
// lanes[l] .. lanes[l + 1] - 1 in order. A segment covering all keys of its
// query tile writes the output; otherwise it writes its unnormalised partial
// (o, max, sum) to slot = segment index, and one merge entry {first slot,
// number of slots, first output row, valid rows} combines the consecutive
// slots of a query tile in slot order.
struct AttnArgs {
  const half *qu, *qv, *kh, *vt, *rk;
  half* out;       // (mp, 1024) heads-flat
  int mp;          // rows of qu/qv/kh and columns of vt
  int pp;          // rows of rk per head
  int tc;          // rk row j <-> relative position r = tc - 1 - j
  const int4* tiles;  // segments
  int ntiles;
  const int* lanes;   // nlanes + 1 segment offsets
  int nlanes;
  half* part_o = nullptr;    // [slot][head][query tile][128 d]: o / sum, f16
  float* part_ml = nullptr;  // [slot][head][query tile][2] (max, sum)
  const int4* merges = nullptr;
  int nmerges = 0;
};
// Workgroup lanes per head for one sequence of length t (a function of t
// only, so a sequence's arithmetic does not depend on the rest of its batch):
// its query tile x key tile units are spread evenly over the lanes.
int attention_lanes(int t);
// Queries per attention work tile (256; 128 with BARK_HIP_ATTN_WAVES=4): the
// unit of the tiles, merges and partial buffers of AttnArgs.
int attention_query_tile();
// q+u and q+v must be pre-multiplied by attention_q_scale() = log2(e)/sqrt(128)
// (the Qkv epilogue does it when EpiArgs::scale is set to this value).
// rel_attention writes the complete query tiles and the partials of split
// ones; rel_attention_merge (a no-op without splits) then writes the rest.
void rel_attention(const AttnArgs& a, hipStream_t stream);
void rel_attention_merge(const AttnArgs& a, hipStream_t stream);
float attention_q_scale();

// ----------------------------------------------------------------- ops --
// LayerNorm over 1024 columns. y16 and/or y32 may be null. With a pending
// residual update `res`, x is first updated in place (x += res) and the norm
// is taken of the updated rows.
void layer_norm(float* x, const float* w, const float* b, half* y16, float* y32,
                int rows, hipStream_t stream, const ResidIn& res = ResidIn());
// y32 = LN_a(x + res) (written), y16 = f16(LN_b(y32)); x itself is not
// updated (the residual stream continues in y32).
void layer_norm2(const float* x, const float* wa, const float* ba, float* y32,
                 const float* wb, const float* bb, half* y16, int rows, hipStream_t stream,
                 const ResidIn& res = ResidIn());
// x += res in place (rows x 1024).
void apply_residual(float* x, int rows, const ResidIn& res, hipStream_t stream);
// out = f16(silu(BN(dwconv9(g)))) with per-row [start, end) frame bounds;
// dw is tap-major [9][1024].
void dwconv_bn_silu(const float* g, const float* dw, const float* bn_a, const float* bn_b,
                    const int2* bounds, half* out, int rows, hipStream_t stream);
void f32_to_f16(const float* x, half* y, size_t n, hipStream_t stream);
// p[0 .. bytes) = 0 with a kernel (no memset node when captured in a graph);
// bytes and p in 16-byte units.
void zero_fill(void* p, size_t bytes, hipStream_t stream);
void f32_to_f16_rows(const float* x, int rows, int cols, half* y, int ldy,
                     hipStream_t stream);
void copy_rows_f32(const float* x, int ldx, float* y, int ldy, int rows, int cols,
                   hipStream_t stream);
// Front end. conv1 (mel (frames, 128) f32 -> (f1, 64, 256), ReLU, rows >= vlen1
// zeroed, f16) fused with the first depthwise 3x3 stride 2 -> (t2, 32, 256) f16,
// rows >= vlen2 zeroed.
void sub_conv1_dw(const float* mel, int frames, const float* w1, const float* b1, int vlen1,
                  const float* wd, const float* bd, int vlen2, half* out, hipStream_t stream);
// depthwise 3x3 stride 2 on (t_in, m_in, 256) -> (t_out, m_out, 256), rows >= vlen zeroed.
void sub_dwconv(const half* in, int t_in, int m_in, const float* w, const float* b,
                half* out, int vlen, hipStream_t stream);

// ------------------------------------------------------------- log-mel --
// Device tables of the log-mel front end (mel.hip): the 512-point window, the
// FFT twiddles (f64: cos then sin of 2 pi k / 512, k < 256), per mel row {first
// bin, bin count, offset into vals} of its nonzero filter range, and the
// filter values of those ranges.
struct MelTables {
  const float* window = nullptr;
  const double* twiddle = nullptr;
  const int* rows = nullptr;
  const float* vals = nullptr;
};
int mel_frames(long n_samples);               // 1 + n / 160
size_t mel_workspace_bytes(long n_samples);   // scratch of mel_features
// features (mel_frames(n) x 128 f32) of a 16 kHz wave, all on `st`
void mel_features(const float* wave, long n_samples, const MelTables& tb, void* workspace, float* out,
                  hipStream_t st);

// ---------------------------------------------------------------- TDT --
// Device buffers of the greedy TDT decoder (tdt.hip): embedding (8193 x 640)
// and biases f32; LSTM (2 layers x 2560 x 640, ih and hh), projection
// (640 x 640) and joint head (8198 x 640) f16; then, per utterance of a batch,
// two control-state buffers, h (2 layers x 2 buffers x 640), c (2 x 640), dec
// (640) and joint partials (2 x 256 float4); token records {id, frame, dur}
// for the whole batch.
struct TdtDev {
  const float* embed = nullptr;
  const half *w_ih = nullptr, *w_hh = nullptr, *proj_w = nullptr, *head_w = nullptr;
  const float *b_ih = nullptr, *b_hh = nullptr, *proj_b = nullptr, *head_b = nullptr;
  int* state = nullptr;
  float *h = nullptr, *c = nullptr, *dec = nullptr, *partials = nullptr;
  uint32_t* tokens = nullptr;
};
constexpr int TDT_PARTIALS = 256;  // joint partials per set (the largest grid); two sets
// bytes per utterance of the batched buffers
constexpr size_t TDT_H_BYTES = 4 * 640 * 4, TDT_C_BYTES = 2 * 640 * 4, TDT_DEC_BYTES = 640 * 4,
                 TDT_PART_BYTES = 2 * TDT_PARTIALS * 16;
int tdt_state_words();  // words of one control state (two buffers per utterance)
int tdt_frame_word();   // index of the frame pointer among the state words
int tdt_done_word();    // index of the `done` flag
int tdt_count_word();   // index of the emitted-token count
int tdt_max_steps(int t_len);
long tdt_max_launches(int t_len);  // launches after which `done` is certain
// reset the control states of `batch` utterances; d_params (device) holds per
// utterance {t_len, first pooler row, first token record, record capacity}
void tdt_begin(const TdtDev& d, const int* d_params, int batch, hipStream_t st);
// queue n launches, each advancing every utterance by the phase its control
// state names; `launches` counts them from tdt_begin (it selects the buffer)
void tdt_launches(const TdtDev& d, const float* pooler, int batch, int n, long& launches, hipStream_t st);
// utterance u's control state after `launches` launches
const int* tdt_current(const TdtDev& d, long launches, int u);

// ---------------------------------------------------------- safetensors --
// One tensor entry of a safetensors header (ingest.hip); begin / end are
// absolute byte offsets in its file.
struct StTensor {
  std::string name, dtype;
  std::vector<int64_t> shape;
  int64_t numel = 0;  // product of shape, checked against overflow when parsed
  uint64_t begin = 0, end = 0;
};
// product of a shape's entries; throws when it overflows (or reaches 2^53)
int64_t shape_elements(const std::vector<int64_t>& shape, const std::string& where);
// the files of a checkpoint: a .safetensors file, or a directory holding
// model.safetensors or model.safetensors.index.json and its shards
std::vector<std::string> safetensors_files(const std::string& path);
std::vector<StTensor> safetensors_header(const std::string& file);
void safetensors_read(const std::string& file, const StTensor& t, void* dst);
// what a checkpoint holds, from its header(s): JSON {release, layout, tensors,
// weights, layers, hidden, ffn, vocab}
std::string safetensors_probe(const std::string& path);

}  // namespace bark
