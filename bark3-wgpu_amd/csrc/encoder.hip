// Host orchestration of the encoder forward and the C ABI (include/bark_hip.h).
//
// Mirrors the reference's GPU encoder driver (src/encoder.rs:412-830 load,
// :1985-2657 encode/encode_pre) and conv front end (src/sub_gpu.rs:574-776),
// re-planned for one MI355X:
//  - weights live in HBM in their compact form (f16 or 4-bit codes + 16-entry
//    f16 tables), fused and permuted once at finalize;
//  - a forward over one or several utterances packs their frames into one row
//    space (each utterance 64-row aligned), so every linear streams its weights
//    once per call whatever the batch;
//  - per block: 4 LayerNorm launches (norm_out fused with the next block's
//    first norm), 9 GEMMs with fused epilogues, 1 attention, 1 dwconv.
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/bark_hip.h"
#include "kernels.h"

namespace bark {
thread_local LaunchTiming g_launch_timing;

namespace {

thread_local std::string g_last_error;

inline int conv_len(int l) { return (l + 2 - 3) / 2 + 1; }  // src/sub.rs:11-13

inline uint16_t f32_to_f16_bits(float v) {
  const half h = (half)v;  // IEEE round-to-nearest-even
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}
inline float f16_bits_to_f32(uint16_t b) {
  half h;
  std::memcpy(&h, &b, 2);
  return (float)h;
}

// src/bark.rs:597-611
float expand_level(uint32_t code, uint32_t k, const uint16_t* levels) {
  if (code == 0) return 0.0f;
  const bool negative = code > k;
  const uint32_t mag = negative ? code - k - 1 : code - 1;
  const float value = mag < k ? f16_bits_to_f32(levels[mag]) : 0.0f;
  return negative ? -value : value;
}

struct HostTensor {
  enum Kind { F32, F16, LUT4 } kind = F32;
  std::vector<int64_t> shape;
  std::vector<float> f32;
  std::vector<uint16_t> f16;
  std::vector<uint8_t> codes;  // rows x cols/2
  std::vector<uint16_t> lut;   // rows x 16
  int64_t rows = 0, cols = 0;
};

// A linear weight on the host side of finalize: f16 bits or codes + tables.
struct HostLinear {
  bool lut4 = false;
  int rows = 0, cols = 0;
  std::vector<uint16_t> w16;
  std::vector<uint8_t> codes;
  std::vector<uint16_t> lut;
};

struct DevLayer {
  GemmWeight qkv, o, ff1a, ff1b, ff2a, ff2b, pw1, pw2;
  float *dw = nullptr, *bn_a = nullptr, *bn_b = nullptr, *bu = nullptr, *bv = nullptr;
  float* ln_w[5] = {};
  float* ln_b[5] = {};
};

// Grow-only device buffer; contents are zeroed whenever it is (re)allocated.
struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// Per-operator GPU timing, the counterpart of the reference's
// BARK3_ENC_PROFILE timestamps (src/encoder/prof.rs:1-127): when enabled, every
// launch is bracketed by two events on its stream; report() aggregates the
// elapsed times per label together with the algorithmic FLOPs and bytes.
struct Profiler {
  struct Op {
    std::string label;
    double flops, bytes;
    hipEvent_t a, b;
  };
  bool on = false;
  std::string only;  // non-empty: time this label only, every ONLY_EVERY-th launch of it
  static constexpr int ONLY_EVERY = 8;
  long only_seen = 0;
  std::vector<hipEvent_t> free_events;
  std::vector<Op> ops;

  hipEvent_t take() {
    if (free_events.empty()) {
      hipEvent_t e;
      BARK_HIP_CHECK(hipEventCreate(&e));
      return e;
    }
    hipEvent_t e = free_events.back();
    free_events.pop_back();
    return e;
  }
  template <class F>
  void run(const char* label, double flops, double bytes, hipStream_t st, F&& f) {
    // Timing a launch costs a few microseconds of dispatch (the events ride on
    // the kernel packet), so a single-label run samples every ONLY_EVERY-th
    // launch: the label's launches are identical work each layer, and the step
    // time around them stays within ~0.5 % of an untimed step.
    if (!on || (!only.empty() && (only != label || only_seen++ % ONLY_EVERY != 0))) {
      f();
      return;
    }
    // the op's kernels carry the events themselves (BARK_LAUNCH)
    Op op{label, flops, bytes, take(), take()};
    g_launch_timing = LaunchTiming{op.a, op.b, 0};
    try {
      f();
    } catch (...) {
      g_launch_timing = LaunchTiming();
      throw;
    }
    const int launched = g_launch_timing.launches;
    g_launch_timing = LaunchTiming();
    if (launched == 0) {  // nothing ran: an empty interval
      BARK_HIP_CHECK(hipEventRecord(op.a, st));
      BARK_HIP_CHECK(hipEventRecord(op.b, st));
    }
    ops.push_back(op);
  }
  std::string report() {
    struct Agg {
      int count = 0;
      double ms = 0, flops = 0, bytes = 0;
    };
    std::map<std::string, Agg> agg;
    for (auto& op : ops) {
      BARK_HIP_CHECK(hipEventSynchronize(op.b));
      float ms = 0;
      BARK_HIP_CHECK(hipEventElapsedTime(&ms, op.a, op.b));
      Agg& g = agg[op.label];
      g.count++;
      g.ms += ms;
      g.flops += op.flops;
      g.bytes += op.bytes;
      free_events.push_back(op.a);
      free_events.push_back(op.b);
    }
    ops.clear();
    std::string out = "{";
    bool first = true;
    for (auto& kv : agg) {
      char buf[256];
      snprintf(buf, sizeof buf, "%s\"%s\":{\"count\":%d,\"ms\":%.6f,\"flops\":%.6e,\"bytes\":%.6e}",
               first ? "" : ",", kv.first.c_str(), kv.second.count, kv.second.ms, kv.second.flops,
               kv.second.bytes);
      out += buf;
      first = false;
    }
    return out + "}";
  }
  ~Profiler() {
    for (auto& op : ops) {
      (void)hipEventDestroy(op.a);
      (void)hipEventDestroy(op.b);
    }
    for (auto e : free_events) (void)hipEventDestroy(e);
  }
};

struct SeqPlan {
  int frames = 0, valid = 0;
  int t = 0;      // encoder frames
  int start = 0;  // first row in the packed row space
};

}  // namespace
}  // namespace bark

using namespace bark;

struct BarkHip {
  int device = 0;
  int n_layers = 24;
  hipStream_t stream = nullptr;
  std::mutex mu;
  // Cross-stream ordering of calls on this handle: every call that queues
  // work records `done` on its stream when it has queued everything, and the
  // next call's stream waits for it first. The workspace buffers are shared
  // by all calls, so a call on another stream must not start before the
  // previous one has finished with them.
  hipEvent_t done = nullptr;
  hipStream_t done_stream = nullptr;
  void order_after_previous(hipStream_t st) {
    if (done_stream && done_stream != st) BARK_HIP_CHECK(hipStreamWaitEvent(st, done, 0));
  }
  void mark_done(hipStream_t st) {
    BARK_HIP_CHECK(hipEventRecord(done, st));
    done_stream = st;
  }
  // runs f (which queues work on st) ordered after the previous call
  template <class F>
  void on_stream(hipStream_t st, F&& f) {
    order_after_previous(st);
    try {
      f();
    } catch (...) {
      (void)hipEventRecord(done, st);  // whatever was queued before the error
      done_stream = st;
      throw;
    }
    mark_done(st);
  }
  // pinned staging of the plan tables (bounds, attention segments, merges,
  // lanes): host memory that lives until the copies reading it have run
  // (tables_copied), so a new packing needs no stream synchronisation
  void* tables_host = nullptr;
  size_t tables_host_cap = 0;
  hipEvent_t tables_copied = nullptr;
  std::map<std::string, HostTensor> staged;
  bool finalized = false;
  bool has_front_end = false;

  std::vector<void*> allocs;  // weights, freed at destroy
  Profiler prof;
  std::vector<int> table_key;  // plan whose row bounds / query tiles are on the device
  // The encode (front end + blocks) as a HIP graph, for short utterances
  // where launching ~370 kernels one by one costs more than running them.
  // Keyed on the packing, the input pointer and ws_gen (bumped by every
  // workspace reallocation, so no baked-in pointer goes stale): the first call
  // with a key runs eagerly, a repeat captures it on cap_stream, later repeats
  // replay it. BARK_HIP_GRAPH=0 turns it off; profiling runs eagerly.
  long ws_gen = 0;
  hipStream_t cap_stream = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  std::vector<long> graph_key, last_key;
  GemmWeight sub_w, proj_w, sub_pw1, sub_pw2;
  // relative_k_proj of every layer stacked (row block l = layer l): the
  // position keys depend on T only, so all layers' relK come from one GEMM.
  GemmWeight relk_all;
  float *sub_b = nullptr, *proj_b = nullptr;
  float *l0w = nullptr, *l0b = nullptr, *l2w = nullptr, *l2b = nullptr, *l3b = nullptr;
  float *l5w = nullptr, *l5b = nullptr, *l6b = nullptr;
  std::vector<DevLayer> layers;

  // log-mel front end: window, twiddles, sparse filterbank, scratch
  DevBuf mel_window, mel_twid, mel_rows, mel_vals, mel_ws, mel_wave, mel_feat;
  bool has_mel = false;

  // greedy TDT decoder: weights (uploaded by finalize when the decoder's
  // tensors were staged), state, and a pinned copy of the state words
  TdtDev tdt;
  bool has_tdt = false;
  DevBuf tdt_state, tdt_h, tdt_c, tdt_dec, tdt_part, tdt_tokens, tdt_pooler, tdt_params;

  void set_mel_filters(const float* filters) {
    constexpr int NB = 257;
    std::vector<float> win(512, 0.0f);
    for (int i = 0; i < 400; ++i) {  // symmetric Hann, as src/mel.rs:28-35 computes it in f32
      const float a = 6.28318530717958647692f * (float)i / 399.0f;
      win[56 + i] = 0.5f * (1.0f - std::cos(a));
    }
    std::vector<double> tw(512);
    for (int k = 0; k < 256; ++k) {
      tw[k] = std::cos(2.0 * M_PI * k / 512.0);
      tw[256 + k] = std::sin(2.0 * M_PI * k / 512.0);
    }
    std::vector<int> rows(3 * MEL);
    std::vector<float> vals;
    for (int m = 0; m < MEL; ++m) {  // the nonzero range of each row (zeros inside add nothing)
      int first = -1, last = -1;
      for (int k = 0; k < NB; ++k)
        if (filters[(size_t)m * NB + k] != 0.0f) {
          if (first < 0) first = k;
          last = k;
        }
      const int count = first < 0 ? 0 : last - first + 1;
      rows[3 * m] = std::max(first, 0);
      rows[3 * m + 1] = count;
      rows[3 * m + 2] = (int)vals.size();
      for (int k = 0; k < count; ++k) vals.push_back(filters[(size_t)m * NB + first + k]);
    }
    ensure(mel_window, win.size() * 4);
    ensure(mel_twid, tw.size() * 8);
    ensure(mel_rows, rows.size() * 4);
    ensure(mel_vals, std::max<size_t>(vals.size(), 1) * 4);
    BARK_HIP_CHECK(hipMemcpy(mel_window.p, win.data(), win.size() * 4, hipMemcpyHostToDevice));
    BARK_HIP_CHECK(hipMemcpy(mel_twid.p, tw.data(), tw.size() * 8, hipMemcpyHostToDevice));
    BARK_HIP_CHECK(hipMemcpy(mel_rows.p, rows.data(), rows.size() * 4, hipMemcpyHostToDevice));
    if (!vals.empty()) BARK_HIP_CHECK(hipMemcpy(mel_vals.p, vals.data(), vals.size() * 4, hipMemcpyHostToDevice));
    has_mel = true;
  }

  void run_mel(const float* d_wave, long n, float* d_out, size_t cap, int32_t* n_frames, int32_t* n_valid,
               hipStream_t st) {
    BARK_REQUIRE(has_mel, "bark_hip_set_mel_filters was not called");
    BARK_REQUIRE(n > 0, "empty wave");
    const int nf = mel_frames(n);
    BARK_REQUIRE(cap >= (size_t)nf * MEL, "features buffer too small");
    ensure(mel_ws, mel_workspace_bytes(n));
    MelTables tb;
    tb.window = mel_window.as<float>();
    tb.twiddle = mel_twid.as<double>();
    tb.rows = mel_rows.as<int>();
    tb.vals = mel_vals.as<float>();
    prof.run("mel", 0, 4.0 * n + 4.0 * nf * MEL * 3, st, [&] { mel_features(d_wave, n, tb, mel_ws.p, d_out, st); });
    if (n_frames) *n_frames = nf;
    if (n_valid) *n_valid = (int32_t)(n / 160);
  }

  // position table rows for pos = pos_t-1 .. -(pos_t-1), f16, plus zero rows
  DevBuf pos;
  int pos_t = 0;
  // rk holds every layer's relative keys for all rows of the position table
  // as of pos_t == relk_t (0: not computed); see encoder_blocks
  int relk_t = 0;

  // workspace
  DevBuf sub16, xn, hid, qu, qv, kh, vt, rk, ao, h, h2, glu, pooler, dump, bounds, tiles;
  DevBuf part;  // split-K partial sums of the residual linears
  DevBuf merges, attn_lanes, attn_po, attn_pml;  // attention work lanes and key-range partials
  DevBuf y2, y3, y4, mel, subf32;

  template <class T>
  T* upload(const T* src, size_t n) {
    void* p = nullptr;
    BARK_HIP_CHECK(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)));
    allocs.push_back(p);
    BARK_HIP_CHECK(hipMemcpy(p, src, n * sizeof(T), hipMemcpyHostToDevice));
    return static_cast<T*>(p);
  }

  void ensure(DevBuf& b, size_t bytes) {
    if (bytes <= b.cap) return;
    if (&b == &bounds || &b == &tiles || &b == &merges || &b == &attn_lanes) table_key.clear();
    BARK_HIP_CHECK(hipDeviceSynchronize());  // any stream may still use the old buffer
    if (b.p) BARK_HIP_CHECK(hipFree(b.p));
    b.p = nullptr;
    b.cap = 0;
    const size_t want = (bytes + 4095) & ~size_t(4095);
    BARK_HIP_CHECK(hipMalloc(&b.p, want));
    ++ws_gen;
    BARK_HIP_CHECK(hipMemset(b.p, 0, want));
    // the fill runs on the null stream, which the library's non-blocking
    // streams do not wait for: finish it before anything is queued after it
    BARK_HIP_CHECK(hipDeviceSynchronize());
    b.cap = want;
  }

  ~BarkHip() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (void* p : allocs) (void)hipFree(p);
    DevBuf* bufs[] = {&pos, &sub16, &xn, &hid, &qu, &qv, &kh, &vt, &rk, &ao, &h, &h2, &glu, &part,
                      &pooler, &dump, &bounds, &tiles, &y2, &y3, &y4, &mel, &subf32,
                      &merges, &attn_lanes, &attn_po, &attn_pml, &mel_window, &mel_twid,
                      &mel_rows, &mel_vals, &mel_ws, &mel_wave, &mel_feat, &tdt_state, &tdt_h,
                      &tdt_c, &tdt_dec, &tdt_part, &tdt_tokens, &tdt_pooler, &tdt_params};
    for (DevBuf* b : bufs)
      if (b->p) (void)hipFree(b->p);
    if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
    if (cap_stream) (void)hipStreamDestroy(cap_stream);
    if (stream) (void)hipStreamDestroy(stream);
    if (done) (void)hipEventDestroy(done);
    if (tables_copied) (void)hipEventDestroy(tables_copied);
    if (tables_host) (void)hipHostFree(tables_host);
  }

  // ------------------------------------------------------------ finalize --
  const HostTensor& need(const std::string& name) {
    auto it = staged.find(name);
    BARK_REQUIRE(it != staged.end(), "missing tensor " + name);
    return it->second;
  }

  std::vector<float> vec_f32(const std::string& name, int64_t n) {
    const HostTensor& t = need(name);
    std::vector<float> out;
    if (t.kind == HostTensor::F32) {
      out = t.f32;
    } else if (t.kind == HostTensor::F16) {
      out.resize(t.f16.size());
      for (size_t i = 0; i < t.f16.size(); ++i) out[i] = f16_bits_to_f32(t.f16[i]);
    } else {
      throw Error{name + ": a 4-bit tensor where f32 values are expected"};
    }
    BARK_REQUIRE((int64_t)out.size() == n,
                 name + ": expected " + std::to_string(n) + " values, got " +
                     std::to_string(out.size()));
    return out;
  }

  HostLinear linear(const std::string& name, int rows, int cols, bool allow_lut4) {
    const HostTensor& t = need(name);
    HostLinear L;
    L.rows = rows;
    L.cols = cols;
    if (t.kind == HostTensor::LUT4) {
      BARK_REQUIRE(allow_lut4, name + ": 4-bit storage is not supported for this tensor");
      BARK_REQUIRE(t.rows == rows && t.cols == cols, name + ": 4-bit tensor has a wrong shape");
      L.lut4 = true;
      L.codes = t.codes;
      L.lut = t.lut;
      return L;
    }
    const int64_t n = (int64_t)rows * cols;
    if (t.kind == HostTensor::F16) {
      BARK_REQUIRE((int64_t)t.f16.size() == n, name + ": wrong element count");
      L.w16 = t.f16;
    } else {
      BARK_REQUIRE((int64_t)t.f32.size() == n, name + ": wrong element count");
      L.w16.resize(n);
      for (int64_t i = 0; i < n; ++i) L.w16[i] = f32_to_f16_bits(t.f32[i]);
    }
    return L;
  }

  GemmWeight to_device(const HostLinear& L) {
    GemmWeight g;
    g.n = L.rows;
    g.k = L.cols;
    if (L.lut4) {
      BARK_REQUIRE(L.cols % 64 == 0, "4-bit weights need a multiple of 64 columns");
      std::vector<uint8_t> sw = L.codes;
      swizzle_codes(sw.data(), sw.size());
      g.codes = upload(sw.data(), sw.size());
      g.swizzled = true;
      g.lut = reinterpret_cast<const half*>(upload(L.lut.data(), L.lut.size()));
    } else {
      g.w16 = reinterpret_cast<const half*>(upload(L.w16.data(), L.w16.size()));
    }
    return g;
  }

  // Rows of several linears stacked (q|k|v, src/encoder.rs:342-402).
  static HostLinear stack(const std::vector<HostLinear>& parts, const std::string& what) {
    HostLinear out;
    out.lut4 = parts[0].lut4;
    out.cols = parts[0].cols;
    for (const auto& p : parts) {
      BARK_REQUIRE(p.lut4 == out.lut4, what + " mixes 4-bit and f16 storage");
      BARK_REQUIRE(p.cols == out.cols, what + ": column mismatch");
      out.rows += p.rows;
      out.w16.insert(out.w16.end(), p.w16.begin(), p.w16.end());
      out.codes.insert(out.codes.end(), p.codes.begin(), p.codes.end());
      out.lut.insert(out.lut.end(), p.lut.begin(), p.lut.end());
    }
    return out;
  }

  // pw1 rows (2048) reordered so each 64-row group is [value 32 | gate 32] of
  // the same 32 output channels: new row 64g+32s+j <- old row 1024s+32g+j.
  static HostLinear interleave_glu(const HostLinear& in) {
    HostLinear out = in;
    const int half_rows = in.rows / 2;
    auto src_row = [&](int nr) {
      const int g = nr / 64, s = (nr % 64) / 32, j = nr % 32;
      return s * half_rows + 32 * g + j;
    };
    for (int nr = 0; nr < in.rows; ++nr) {
      const int orow = src_row(nr);
      if (in.lut4) {
        const size_t cb = in.cols / 2;
        std::memcpy(&out.codes[nr * cb], &in.codes[orow * cb], cb);
        std::memcpy(&out.lut[nr * 16], &in.lut[orow * 16], 32);
      } else {
        std::memcpy(&out.w16[(size_t)nr * in.cols], &in.w16[(size_t)orow * in.cols],
                    (size_t)in.cols * 2);
      }
    }
    return out;
  }

  float* f32_dev(const std::string& name, int64_t n) {
    auto v = vec_f32(name, n);
    return upload(v.data(), v.size());
  }

  void finalize() {
    BARK_REQUIRE(!finalized, "finalize called twice");
    sub_w = to_device(linear("encoder.subsampling.linear.weight", 1024, 4096, true));
    sub_b = f32_dev("encoder.subsampling.linear.bias", 1024);
    proj_w = to_device(linear("encoder_projector.weight", PROJ, HIDDEN, false));
    proj_b = f32_dev("encoder_projector.bias", PROJ);
    layers.resize(n_layers);
    std::vector<HostLinear> relk;
    for (int l = 0; l < n_layers; ++l) {
      const std::string p = "encoder.layers." + std::to_string(l) + ".";
      DevLayer& L = layers[l];
      L.qkv = to_device(stack({linear(p + "self_attn.q_proj.weight", 1024, 1024, true),
                               linear(p + "self_attn.k_proj.weight", 1024, 1024, true),
                               linear(p + "self_attn.v_proj.weight", 1024, 1024, true)},
                              "fused q/k/v"));
      relk.push_back(linear(p + "self_attn.relative_k_proj.weight", 1024, 1024, true));
      L.o = to_device(linear(p + "self_attn.o_proj.weight", 1024, 1024, true));
      L.ff1a = to_device(linear(p + "feed_forward1.linear1.weight", 4096, 1024, true));
      L.ff1b = to_device(linear(p + "feed_forward1.linear2.weight", 1024, 4096, true));
      L.ff2a = to_device(linear(p + "feed_forward2.linear1.weight", 4096, 1024, true));
      L.ff2b = to_device(linear(p + "feed_forward2.linear2.weight", 1024, 4096, true));
      L.pw1 = to_device(interleave_glu(linear(p + "conv.pointwise_conv1.weight", 2048, 1024, true)));
      L.pw2 = to_device(linear(p + "conv.pointwise_conv2.weight", 1024, 1024, true));
      {  // depthwise weights as f16-rounded values (the reference stores f16),
         // tap-major [9][1024] so a thread's 4 channels of one tap are one load
        auto dw = vec_f32(p + "conv.depthwise_conv.weight", 1024 * 9);
        std::vector<float> tap(dw.size());
        for (int c = 0; c < 1024; ++c)
          for (int i = 0; i < 9; ++i) tap[(size_t)i * 1024 + c] = f16_bits_to_f32(f32_to_f16_bits(dw[(size_t)c * 9 + i]));
        L.dw = upload(tap.data(), tap.size());
      }
      {  // BatchNorm fold a = w/sqrt(var+1e-5), b = bias - mean*a (src/encoder.rs:546-557)
        auto w = vec_f32(p + "conv.norm.weight", 1024), b = vec_f32(p + "conv.norm.bias", 1024);
        auto m = vec_f32(p + "conv.norm.running_mean", 1024);
        auto v = vec_f32(p + "conv.norm.running_var", 1024);
        std::vector<float> a(1024), bb(1024);
        for (int c = 0; c < 1024; ++c) {
          a[c] = w[c] / std::sqrt(v[c] + 1e-5f);
          bb[c] = b[c] - m[c] * a[c];
        }
        L.bn_a = upload(a.data(), a.size());
        L.bn_b = upload(bb.data(), bb.size());
      }
      const char* ln_names[5] = {"norm_feed_forward1", "norm_self_att", "norm_conv",
                                 "norm_feed_forward2", "norm_out"};
      for (int i = 0; i < 5; ++i) {
        L.ln_w[i] = f32_dev(p + ln_names[i] + ".weight", 1024);
        L.ln_b[i] = f32_dev(p + ln_names[i] + ".bias", 1024);
      }
      L.bu = f32_dev(p + "self_attn.bias_u", 1024);
      L.bv = f32_dev(p + "self_attn.bias_v", 1024);
    }
    relk_all = to_device(stack(relk, "relative_k_proj"));
    // conv front end (optional: encode_sub does not need it)
    const std::string s = "encoder.subsampling.layers.";
    has_front_end = staged.count(s + "0.weight") > 0;
    if (has_front_end) {
      l0w = f32_dev(s + "0.weight", 256 * 9);
      l0b = f32_dev(s + "0.bias", 256);
      l2w = f32_dev(s + "2.weight", 256 * 9);
      l2b = f32_dev(s + "2.bias", 256);
      sub_pw1 = to_device(linear(s + "3.weight", 256, 256, false));
      l3b = f32_dev(s + "3.bias", 256);
      l5w = f32_dev(s + "5.weight", 256 * 9);
      l5b = f32_dev(s + "5.bias", 256);
      sub_pw2 = to_device(linear(s + "6.weight", 256, 256, false));
      l6b = f32_dev(s + "6.bias", 256);
    }
    has_tdt = staged.count("decoder.embedding.weight") > 0;
    if (has_tdt) finalize_tdt();
    staged.clear();
    finalized = true;
  }

  // TdtDecoder::from_source (src/tdt.rs:130-162): embedding f32, LSTM /
  // projection / head weights rounded to f16 (pack16), layer 0 and 1 joined.
  void finalize_tdt() {
    constexpr int DH = 640, GS = 4 * DH, NV = 8193, NR = 8198;
    tdt.embed = f32_dev("decoder.embedding.weight", (int64_t)NV * DH);
    auto joined16 = [&](const std::string& a, const std::string& b) {
      HostLinear la = linear(a, GS, DH, false), lb = linear(b, GS, DH, false);
      la.w16.insert(la.w16.end(), lb.w16.begin(), lb.w16.end());
      return reinterpret_cast<const half*>(upload(la.w16.data(), la.w16.size()));
    };
    auto joined32 = [&](const std::string& a, const std::string& b) {
      auto va = vec_f32(a, GS), vb = vec_f32(b, GS);
      va.insert(va.end(), vb.begin(), vb.end());
      return upload(va.data(), va.size());
    };
    const std::string d = "decoder.lstm.";
    tdt.w_ih = joined16(d + "weight_ih_l0", d + "weight_ih_l1");
    tdt.w_hh = joined16(d + "weight_hh_l0", d + "weight_hh_l1");
    tdt.b_ih = joined32(d + "bias_ih_l0", d + "bias_ih_l1");
    tdt.b_hh = joined32(d + "bias_hh_l0", d + "bias_hh_l1");
    HostLinear pw = linear("decoder.decoder_projector.weight", DH, DH, false);
    tdt.proj_w = reinterpret_cast<const half*>(upload(pw.w16.data(), pw.w16.size()));
    tdt.proj_b = f32_dev("decoder.decoder_projector.bias", DH);
    HostLinear hw = linear("joint.head.weight", NR, DH, false);
    tdt.head_w = reinterpret_cast<const half*>(upload(hw.w16.data(), hw.w16.size()));
    tdt.head_b = f32_dev("joint.head.bias", NR);
  }

  // Greedy TDT decoding of `batch` device poolers (TdtDecoder::decode,
  // src/tdt.rs:318-414; GpuTdtDecoder::decode_async, src/tdt_gpu.rs:206-300):
  // utterance u has t[u] frames of 640 f32 from row rows[u] of d_pooler. Every
  // launch advances all utterances; launches are queued in chunks, after each
  // chunk only the control states come back, and decoding ends when every
  // utterance is done. Returns the token counts; utterance u's {id, frame, dur}
  // records start at record first[u] of tdt_tokens.
  std::vector<int> tdt_decode(const float* d_pooler, const int* rows, const int* t, int batch,
                              std::vector<size_t>& first, hipStream_t st) {
    BARK_REQUIRE(finalized, "decode before finalize");
    BARK_REQUIRE(has_tdt, "no TDT decoder tensors were set before finalize");
    BARK_REQUIRE(batch >= 1 && batch <= 65535, "batch out of range");
    std::vector<int> params(4 * (size_t)batch);
    first.assign(batch, 0);
    size_t records = 0;
    long max_launches = 0;
    int max_t = 0;
    for (int u = 0; u < batch; ++u) {
      BARK_REQUIRE(t[u] >= 0 && t[u] <= (1 << 24), "t_len out of range");
      BARK_REQUIRE(t[u] == 0 || d_pooler, "null pooler");
      const int cap = t[u] ? tdt_max_steps(t[u]) : 0;
      params[4 * u] = t[u];
      params[4 * u + 1] = rows[u];
      params[4 * u + 2] = (int)records;
      params[4 * u + 3] = cap;
      first[u] = records;
      records += (size_t)cap;
      BARK_REQUIRE(records < (1u << 31), "too many frames for one decode");
      if (t[u]) max_launches = std::max(max_launches, tdt_max_launches(t[u]));
      max_t = std::max(max_t, t[u]);
    }
    std::vector<int> counts(batch, 0);
    if (max_launches == 0) return counts;  // every pooler empty (src/tdt_gpu.rs:211-216)
    const size_t words = (size_t)tdt_state_words();
    ensure(tdt_state, (size_t)batch * 2 * words * 4);
    ensure(tdt_h, (size_t)batch * TDT_H_BYTES);
    ensure(tdt_c, (size_t)batch * TDT_C_BYTES);
    ensure(tdt_dec, (size_t)batch * TDT_DEC_BYTES);
    ensure(tdt_part, (size_t)batch * TDT_PART_BYTES);
    ensure(tdt_params, params.size() * 4);
    ensure(tdt_tokens, std::max<size_t>(records, 1) * 12);
    TdtDev d = tdt;
    d.state = tdt_state.as<int>();
    d.h = tdt_h.as<float>();
    d.c = tdt_c.as<float>();
    d.dec = tdt_dec.as<float>();
    d.partials = tdt_part.as<float>();
    d.tokens = tdt_tokens.as<uint32_t>();
    BARK_HIP_CHECK(hipMemcpyAsync(tdt_params.p, params.data(), params.size() * 4, hipMemcpyHostToDevice, st));
    tdt_begin(d, tdt_params.as<int>(), batch, st);
    // per token step: joint head, both LSTM layers and the projection (f16)
    const double step_bytes = 2.0 * 640 * (8198 + 4 * 2560 + 640);
    std::vector<int> host((size_t)batch * 2 * words);
    long launches = 0, chunk = std::max(16, max_t / 2);
    bool all_done = false;
    while (true) {
      const int n = (int)std::min(chunk, max_launches - launches);
      prof.run("tdt_decode", 0, step_bytes * n / 4 * batch, st,
               [&] { tdt_launches(d, d_pooler, batch, n, launches, st); });
      BARK_HIP_CHECK(hipMemcpyAsync(host.data(), d.state, host.size() * 4, hipMemcpyDeviceToHost, st));
      BARK_HIP_CHECK(hipStreamSynchronize(st));
      // the rest at the rate seen so far (launches per frame), for the utterance furthest behind
      all_done = true;
      long rest = 0;
      for (int u = 0; u < batch; ++u) {
        const int* cur = host.data() + (tdt_current(d, launches, u) - d.state);
        if (cur[tdt_done_word()]) continue;
        all_done = false;
        const int frame = cur[tdt_frame_word()];
        rest = std::max(rest, (long)((double)launches / std::max(frame, 1) * (t[u] - frame)));
      }
      if (all_done || launches >= max_launches) break;
      chunk = std::max(16L, rest + 8);
    }
    BARK_REQUIRE(all_done, "TDT decoding did not finish within the step guard");
    for (int u = 0; u < batch; ++u)
      counts[u] = (host.data() + (tdt_current(d, launches, u) - d.state))[tdt_count_word()];
    return counts;
  }

  // decode and copy every utterance's records to `tokens` back to back
  void tdt_decode_copy(const float* d_pooler, const int* rows, const int* t, int batch, uint32_t* tokens, size_t cap,
                       int32_t* n_tokens, hipStream_t st) {
    std::vector<size_t> first;
    const std::vector<int> counts = tdt_decode(d_pooler, rows, t, batch, first, st);
    size_t total = 0;
    for (int u = 0; u < batch; ++u) {
      if (n_tokens) n_tokens[u] = counts[u];
      total += (size_t)counts[u];
    }
    BARK_REQUIRE(total <= cap, "token buffer too small: " + std::to_string(total) + " tokens");
    size_t off = 0;
    for (int u = 0; u < batch; ++u) {
      if (counts[u] > 0) {
        BARK_REQUIRE(tokens, "null token buffer");
        BARK_HIP_CHECK(hipMemcpyAsync(tokens + 3 * off, tdt_tokens.as<uint32_t>() + 3 * first[u],
                                      (size_t)counts[u] * 12, hipMemcpyDeviceToHost, st));
      }
      off += (size_t)counts[u];
    }
    BARK_HIP_CHECK(hipStreamSynchronize(st));
  }

  // ------------------------------------------------------- position table --
  // src/encoder.rs:228-245 evaluated on the host with the platform libm, as
  // the reference does; rows cover pos = pos_t-1 .. -(pos_t-1) so any T <=
  // pos_t is a contiguous sub-range starting at row pos_t - T.
  void ensure_pos(int t) {
    if (t <= pos_t) return;
    const int tt = std::max(t, 256);
    const int rows = 2 * tt - 1;
    std::vector<float> inv(HIDDEN / 2);
    for (int i = 0; i < HIDDEN / 2; ++i)
      inv[i] = 1.0f / std::pow(10000.0f, (2.0f * (float)i) / (float)HIDDEN);
    std::vector<uint16_t> tab((size_t)(rows + 128) * HIDDEN, 0);
    const int nth = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    for (int w = 0; w < nth; ++w)
      th.emplace_back([&, w] {
        for (int pi = w; pi < rows; pi += nth) {
          const float posv = (float)((rows - 1) / 2 - pi);
          uint16_t* row = &tab[(size_t)pi * HIDDEN];
          for (int i = 0; i < HIDDEN / 2; ++i) {
            const float f = posv * inv[i];
            row[2 * i] = f32_to_f16_bits(std::sin(f));
            row[2 * i + 1] = f32_to_f16_bits(std::cos(f));
          }
        }
      });
    for (auto& x : th) x.join();
    ensure(pos, tab.size() * 2);
    BARK_HIP_CHECK(hipMemcpy(pos.p, tab.data(), tab.size() * 2, hipMemcpyHostToDevice));
    pos_t = tt;
  }

  // ------------------------------------------------------------- forward --
  struct Plan {
    std::vector<SeqPlan> seqs;
    int mp = 0;  // packed rows (multiple of 64)
    int tc = 0;  // longest sequence: relK covers |q-k| < tc
  };

  static Plan make_plan(const int32_t* frames, const int32_t* valid, const int32_t* tlen,
                        int batch) {
    Plan pl;
    int row = 0;
    for (int i = 0; i < batch; ++i) {
      SeqPlan s;
      if (frames) {
        BARK_REQUIRE(frames[i] >= 1, "n_frames must be >= 1");
        s.frames = frames[i];
        s.valid = valid ? valid[i] : frames[i];
        s.t = conv_len(conv_len(conv_len(s.frames)));
      } else {
        s.t = tlen[i];
      }
      BARK_REQUIRE(s.t >= 1, "sequence length must be >= 1");
      s.start = row;
      row += round_up(s.t, 64);
      pl.tc = std::max(pl.tc, s.t);
      pl.seqs.push_back(s);
    }
    pl.mp = row;
    return pl;
  }

  void ensure_workspace(const Plan& pl) {
    const size_t mp = pl.mp;
    ensure(sub16, mp * 4096 * 2);
    ensure(xn, mp * HIDDEN * 2);
    ensure(hid, mp * FFN * 2);
    ensure(qu, HEADS * mp * HDIM * 2);
    ensure(qv, HEADS * mp * HDIM * 2);
    ensure(kh, HEADS * mp * HDIM * 2);
    ensure(vt, HEADS * mp * HDIM * 2);
    ensure_pos(pl.tc);
    {  // relative keys of every position of the table (encoder_blocks)
      const void* old = rk.p;
      ensure(rk, (size_t)n_layers * HEADS * round_up(2 * pos_t - 1, 64) * HDIM * 2);
      if (rk.p != old) relk_t = 0;
    }
    ensure(ao, mp * HIDDEN * 2);
    ensure(h, mp * HIDDEN * 4);
    ensure(h2, mp * HIDDEN * 4);
    ensure(glu, mp * HIDDEN * 4);
    ensure(part, (size_t)std::max(residual_splits(HIDDEN, HIDDEN), residual_splits(HIDDEN, FFN)) * mp *
                     HIDDEN * 4);
    ensure(pooler, mp * PROJ * 4);
    ensure(bounds, mp * sizeof(int2));
    std::vector<int4> tl, ml;
    std::vector<int> ll;
    attention_tables(pl, tl, ll, ml);
    ensure(tiles, tl.size() * sizeof(int4));
    ensure(attn_lanes, ll.size() * sizeof(int));
    ensure(merges, std::max<size_t>(ml.size(), 1) * sizeof(int4));
    if (!ml.empty()) {
      ensure(attn_po, tl.size() * HEADS * attention_query_tile() * HDIM * 2);
      ensure(attn_pml, tl.size() * HEADS * attention_query_tile() * 2 * 4);
    }
  }

  // Attention work list. Per sequence, its query tile x key tile units (in
  // query tile, then key tile order) are cut evenly over attention_lanes(t)
  // workgroup lanes; a lane's range becomes one segment per query tile it
  // touches, so the pieces of one query tile are consecutive segments, and a
  // merge entry joins them when there is more than one.
  static void attention_tables(const Plan& pl, std::vector<int4>& tl, std::vector<int>& ll,
                               std::vector<int4>& ml) {
    const int bq = attention_query_tile();
    for (const auto& s : pl.seqs) {
      const int ntk = (s.t + 63) / 64, nqt = (s.t + bq - 1) / bq;
      const long units = (long)nqt * ntk;
      const int lanes = attention_lanes(s.t);
      const size_t first = tl.size();
      for (int l = 0; l < lanes; ++l) {
        ll.push_back((int)tl.size());
        const long u1 = units * (l + 1) / lanes;
        for (long u = units * l / lanes; u < u1;) {
          const int qi = (int)(u / ntk), kb = (int)(u % ntk);
          const int ke = (int)std::min<long>(ntk, kb + (u1 - u));
          tl.push_back(make_int4(s.start, s.t, qi * bq, kb | (ke << 16)));
          u += ke - kb;
        }
      }
      for (size_t i = first; i < tl.size();) {
        size_t j = i + 1;
        while (j < tl.size() && tl[j].z == tl[i].z) ++j;
        if (j - i > 1) ml.push_back(make_int4((int)i, (int)(j - i), s.start + tl[i].z, std::min(bq, s.t - tl[i].z)));
        i = j;
      }
    }
    ll.push_back((int)tl.size());
  }

  // Row bounds for the depthwise conv and query tiles for attention.
  void upload_tables(const Plan& pl, hipStream_t st) {
    std::vector<int> key{pl.mp};
    for (const auto& s : pl.seqs) {
      key.push_back(s.start);
      key.push_back(s.t);
    }
    if (key == table_key) return;  // same packing as the previous call
    std::vector<int2> b(pl.mp);
    for (int r = 0; r < pl.mp; ++r) b[r] = make_int2(r, r + 1);
    for (const auto& s : pl.seqs)
      for (int r = s.start; r < s.start + s.t; ++r) b[r] = make_int2(s.start, s.start + s.t);
    std::vector<int4> tl, ml;
    std::vector<int> ll;
    attention_tables(pl, tl, ll, ml);
    // the four tables back to back in pinned host memory; the previous
    // tables' copies must have read theirs before it is overwritten (they
    // normally finished long ago: this wait is not a stream synchronisation)
    const size_t nb = b.size() * sizeof(int2), nt = tl.size() * sizeof(int4), nm = ml.size() * sizeof(int4),
                 nl = ll.size() * sizeof(int);
    const size_t total = nb + nt + nm + nl;
    BARK_HIP_CHECK(hipEventSynchronize(tables_copied));
    if (total > tables_host_cap) {
      if (tables_host) BARK_HIP_CHECK(hipHostFree(tables_host));
      tables_host = nullptr;
      tables_host_cap = 0;
      BARK_HIP_CHECK(hipHostMalloc(&tables_host, total, hipHostMallocDefault));
      tables_host_cap = total;
    }
    char* hp = static_cast<char*>(tables_host);
    std::memcpy(hp, b.data(), nb);
    std::memcpy(hp + nb, tl.data(), nt);
    if (nm) std::memcpy(hp + nb + nt, ml.data(), nm);
    std::memcpy(hp + nb + nt + nm, ll.data(), nl);
    BARK_HIP_CHECK(hipMemcpyAsync(bounds.p, hp, nb, hipMemcpyHostToDevice, st));
    BARK_HIP_CHECK(hipMemcpyAsync(tiles.p, hp + nb, nt, hipMemcpyHostToDevice, st));
    if (nm) BARK_HIP_CHECK(hipMemcpyAsync(merges.p, hp + nb + nt, nm, hipMemcpyHostToDevice, st));
    BARK_HIP_CHECK(hipMemcpyAsync(attn_lanes.p, hp + nb + nt + nm, nl, hipMemcpyHostToDevice, st));
    BARK_HIP_CHECK(hipEventRecord(tables_copied, st));
    ntiles = (int)tl.size();
    nlanes = (int)ll.size() - 1;
    nmerges = (int)ml.size();
    nparts = 0;
    for (const auto& m : ml) nparts += m.y;
    table_key = key;
  }
  int ntiles = 0, nlanes = 0, nmerges = 0, nparts = 0;

  // Algorithmic bytes of a linear's weight operand.
  static double weight_bytes(const GemmWeight& w) {
    return w.lut4() ? (double)w.n * w.k / 2 + 32.0 * w.n : 2.0 * w.n * w.k;
  }

  // One profiled GEMM: flops = 2*m_real*N*K, bytes = weights + A + output.
  void gemm_op(const char* label, const half* A, int lda, int M, int m_real, const GemmWeight& W,
               Epi epi, const EpiArgs& e, double out_bytes_per_row, hipStream_t st) {
    const double flops = 2.0 * m_real * W.n * W.k;
    const double bytes = weight_bytes(W) + 2.0 * m_real * W.k + out_bytes_per_row * m_real;
    prof.run(label, flops, bytes, st, [&] { gemm(A, lda, M, W, epi, e, st); });
  }

  // A residual linear (N = 1024) as split-K partial sums into `part`; the
  // returned update is applied by the LayerNorm that follows it.
  ResidIn resid_op(const char* label, const half* A, int lda, int M, int m_real, const GemmWeight& W,
                   float scale, hipStream_t st) {
    const int splits = residual_splits(W.n, W.k);
    const double flops = 2.0 * m_real * W.n * W.k;
    const double bytes = weight_bytes(W) + 2.0 * m_real * W.k + 4.0 * splits * m_real * W.n;
    prof.run(label, flops, bytes, st,
             [&] { gemm_split(A, lda, M, W, splits, part.as<float>(), HIDDEN, st); });
    ResidIn r;
    r.part = part.as<float>();
    r.splits = splits;
    r.stride = (size_t)M * HIDDEN;
    r.scale = scale;
    return r;
  }

  // conv front end of one utterance into rows [s.start, s.start+s.t) of sub16.
  void front_end(const float* d_mel, const SeqPlan& s, hipStream_t st) {
    BARK_REQUIRE(has_front_end, "the conv subsampling weights were not loaded");
    const int f1 = conv_len(s.frames), t2 = conv_len(f1), t3 = conv_len(t2);
    int vlen = conv_len(std::max(s.valid, 1));
    const double p1 = (double)f1 * 64, p2 = (double)t2 * 32, p3 = (double)t3 * 16;
    const int vlen1 = std::min(vlen, f1);
    vlen = conv_len(vlen);
    prof.run("fe_conv1_dw", 2.0 * 9 * 256 * (p1 + p2), 4.0 * s.frames * MEL + 2.0 * 256 * p2, st, [&] {
      sub_conv1_dw(d_mel, s.frames, l0w, l0b, vlen1, l2w, l2b, std::min(vlen, t2), y2.as<half>(), st);
    });
    EpiArgs e1;
    e1.out_f16 = y3.as<half>();
    e1.ldo = SUB_CH;
    e1.bias = l3b;
    gemm_op("fe_pointwise", y2.as<half>(), SUB_CH, t2 * 32, t2 * 32, sub_pw1, Epi::BiasReluF16, e1,
            2.0 * SUB_CH, st);
    vlen = conv_len(vlen);
    prof.run("fe_dwconv", 2.0 * 9 * 256 * p3, 2.0 * 256 * (p2 + p3), st, [&] {
      sub_dwconv(y3.as<half>(), t2, 32, l5w, l5b, y4.as<half>(), std::min(vlen, t3), st);
    });
    EpiArgs e2;
    e2.out_f16 = sub16.as<half>() + (size_t)s.start * 4096;
    e2.ldo = 4096;
    e2.bias = l6b;
    gemm_op("fe_pointwise", y4.as<half>(), SUB_CH, t3 * 16, t3 * 16, sub_pw2, Epi::FlattenReluF16, e2,
            2.0 * SUB_CH, st);
  }

  void ensure_front_end(const Plan& pl) {
    size_t n2 = 0, n4 = 0;
    for (const auto& s : pl.seqs) {
      const int f1 = conv_len(s.frames), t2 = conv_len(f1), t3 = conv_len(t2);
      n2 = std::max(n2, (size_t)t2 * 32 * SUB_CH);
      n4 = std::max(n4, (size_t)t3 * 16 * SUB_CH);
    }
    ensure(y2, n2 * 2);
    ensure(y3, n2 * 2);
    ensure(y4, n4 * 2);
  }

  // The blocks + projector over the packed rows in sub16 (pooler rows out).
  void encoder_blocks(const Plan& pl, int dump_layer, hipStream_t st) {
    const int mp = pl.mp, tc = pl.tc, prows = 2 * tc - 1;
    int mr = 0;  // real frames (algorithmic work excludes alignment rows)
    double attn_flops = 0;
    for (const auto& q : pl.seqs) {
      mr += q.t;
      attn_flops += 6144.0 * q.t * q.t;  // content + in-band position + AV
    }
    float* hc = h.as<float>();
    float* ha = h2.as<float>();
    half* xnp = xn.as<half>();
    const double ln_bytes = (double)mr * HIDDEN * (4 + 2);

    EpiArgs es;  // sub linear + bias -> h
    es.out_f32 = hc;
    es.ldo = HIDDEN;
    es.bias = sub_b;
    gemm_op("sub_linear", sub16.as<half>(), 4096, mp, mr, sub_w, Epi::StoreF32, es, 4.0 * HIDDEN, st);

    // Relative keys rk[l][h][r][d] = (pos[r] . W_relk[l]^T) for every row r of
    // the position table (positions pos_t-1 .. -(pos_t-1)): they depend on the
    // weights and the table only, so one GEMM per new table length serves
    // every later encode; a sequence set whose longest length is tc reads the
    // rows of positions tc-1 .. -(tc-1), which start at row pos_t - tc. A
    // recomputation changes the offsets a captured graph holds, so it counts
    // as a workspace change (ws_gen).
    const int ppa = round_up(2 * pos_t - 1, 64);  // rk rows per head
    if (relk_t != pos_t) {
      EpiArgs e;
      e.rk = rk.as<half>();
      e.pp = ppa;
      const int rows = 2 * pos_t - 1;
      gemm_op("relk", pos.as<half>(), HIDDEN, rows, rows, relk_all, Epi::RelK, e, 2.0 * HIDDEN * n_layers, st);
      relk_t = pos_t;
      ++ws_gen;
    }
    for (int l = 0; l < n_layers; ++l) {
      const DevLayer& L = layers[l];
      if (l == 0)
        prof.run("layernorm", 0, ln_bytes, st,
                 [&] { layer_norm(hc, L.ln_w[0], L.ln_b[0], xnp, nullptr, mp, st); });
      // ---- FF1: h += 0.5 * W2 silu(W1 LN(h)); the residual add happens in the next LN
      EpiArgs e;
      e.out_f16 = hid.as<half>();
      e.ldo = FFN;
      gemm_op("ff_up_silu", xnp, HIDDEN, mp, mr, L.ff1a, Epi::Silu, e, 2.0 * FFN, st);
      ResidIn res = resid_op("ff_down_resid", hid.as<half>(), FFN, mp, mr, L.ff1b, 0.5f, st);
      // ---- attention
      prof.run("layernorm_resid", 0, ln_bytes + 4.0 * (res.splits + 1) * mr * HIDDEN, st,
               [&] { layer_norm(hc, L.ln_w[1], L.ln_b[1], xnp, nullptr, mp, st, res); });
      e = EpiArgs();
      e.qu = qu.as<half>();
      e.qv = qv.as<half>();
      e.kh = kh.as<half>();
      e.vt = vt.as<half>();
      e.bu = L.bu;
      e.bv = L.bv;
      e.mp = mp;
      e.scale = attention_q_scale();
      gemm_op("qkv_heads", xnp, HIDDEN, mp, mr, L.qkv, Epi::Qkv, e, 2.0 * 4096, st);
      AttnArgs aa{qu.as<half>(), qv.as<half>(), kh.as<half>(), vt.as<half>(),
                  rk.as<half>() + ((size_t)l * HEADS * ppa + (size_t)(pos_t - tc)) * HDIM,
                  ao.as<half>(), mp, ppa, tc, tiles.as<int4>(), ntiles, attn_lanes.as<int>(), nlanes,
                  attn_po.as<half>(), attn_pml.as<float>(), merges.as<int4>(), nmerges};
      prof.run("rel_attention", attn_flops, 2.0 * mr * HIDDEN * 5 + 2.0 * prows * HIDDEN, st,
               [&] { rel_attention(aa, st); });
      if (nmerges)  // partial (o, max, sum) of every split query tile -> heads-flat f16
        prof.run("attn_merge", 0, (double)nparts * HEADS * attention_query_tile() * (HDIM * 2 + 8) + 2.0 * mr * HIDDEN, st,
                 [&] { rel_attention_merge(aa, st); });
      res = resid_op("attn_out_resid", ao.as<half>(), HIDDEN, mp, mr, L.o, 1.0f, st);
      // ---- conv module
      prof.run("layernorm_resid", 0, ln_bytes + 4.0 * (res.splits + 1) * mr * HIDDEN, st,
               [&] { layer_norm(hc, L.ln_w[2], L.ln_b[2], xnp, nullptr, mp, st, res); });
      e = EpiArgs();
      e.out_f32 = glu.as<float>();
      e.ldo = HIDDEN;
      gemm_op("pw1_glu", xnp, HIDDEN, mp, mr, L.pw1, Epi::Glu, e, 4.0 * HIDDEN, st);
      prof.run("dwconv_bn_silu", 2.0 * 9 * mr * HIDDEN, (double)mr * HIDDEN * 6 + 9 * HIDDEN * 4.0, st, [&] {
        dwconv_bn_silu(glu.as<float>(), L.dw, L.bn_a, L.bn_b, bounds.as<int2>(), xnp, mp, st);
      });
      res = resid_op("pw2_resid", xnp, HIDDEN, mp, mr, L.pw2, 1.0f, st);
      // ---- FF2
      prof.run("layernorm_resid", 0, ln_bytes + 4.0 * (res.splits + 1) * mr * HIDDEN, st,
               [&] { layer_norm(hc, L.ln_w[3], L.ln_b[3], xnp, nullptr, mp, st, res); });
      e = EpiArgs();
      e.out_f16 = hid.as<half>();
      e.ldo = FFN;
      gemm_op("ff_up_silu", xnp, HIDDEN, mp, mr, L.ff2a, Epi::Silu, e, 2.0 * FFN, st);
      res = resid_op("ff_down_resid", hid.as<half>(), FFN, mp, mr, L.ff2b, 0.5f, st);
      if (l == dump_layer) {  // the pre-norm residual of this block
        apply_residual(hc, mp, res, st);
        res = ResidIn();
        ensure(dump, (size_t)mp * HIDDEN * 4);
        copy_rows_f32(hc, HIDDEN, dump.as<float>(), HIDDEN, mp, HIDDEN, st);
      }
      // ---- norm_out (fused with the next block's first LayerNorm)
      const double rb = 4.0 * (res.splits ? res.splits : 0) * mr * HIDDEN;
      if (l + 1 < n_layers) {
        const DevLayer& N = layers[l + 1];
        prof.run("layernorm_pair", 0, (double)mr * HIDDEN * (4 + 4 + 2) + rb, st, [&] {
          layer_norm2(hc, L.ln_w[4], L.ln_b[4], ha, N.ln_w[0], N.ln_b[0], xnp, mp, st, res);
        });
      } else {
        prof.run("layernorm_resid", 0, (double)mr * HIDDEN * (4 + 4 + 2) + rb, st,
                 [&] { layer_norm(hc, L.ln_w[4], L.ln_b[4], xnp, ha, mp, st, res); });
      }
      std::swap(hc, ha);
    }
    EpiArgs ep;
    ep.out_f32 = pooler.as<float>();
    ep.ldo = PROJ;
    ep.bias = proj_b;
    gemm_op("projector", xnp, HIDDEN, mp, mr, proj_w, Epi::StoreF32, ep, 4.0 * PROJ, st);
  }

  // Shared body of the mel-input entry points; pooler rows of sequence i are
  // written to out + (sum of earlier t) * 640 with `kind` host or device.
  // out == nullptr leaves the poolers in the workspace (sequence i at row
  // rows_out[i].first, rows_out[i].second rows) for a decode that follows.
  // body(stream) queues one encode; see graph_exec for when it is captured.
  template <class F>
  void run_graphed(const std::vector<long>& key, F&& body, hipStream_t st) {
    static const bool enabled = [] {
      const char* e = getenv("BARK_HIP_GRAPH");
      return !(e && atoi(e) == 0);
    }();
    if (!enabled || prof.on) {
      body(st);
      return;
    }
    if (graph_exec && key == graph_key) {
      BARK_HIP_CHECK(hipGraphLaunch(graph_exec, st));
      return;
    }
    if (key != last_key) {  // a new packing: eager (most are never repeated)
      last_key = key;
      body(st);
      return;
    }
    if (!cap_stream) BARK_HIP_CHECK(hipStreamCreateWithFlags(&cap_stream, hipStreamNonBlocking));
    if (graph_exec) {
      BARK_HIP_CHECK(hipGraphExecDestroy(graph_exec));
      graph_exec = nullptr;
      graph_key.clear();
    }
    hipGraph_t g = nullptr;
    BARK_HIP_CHECK(hipStreamBeginCapture(cap_stream, hipStreamCaptureModeThreadLocal));
    try {
      body(cap_stream);
    } catch (...) {
      (void)hipStreamEndCapture(cap_stream, &g);
      if (g) (void)hipGraphDestroy(g);
      throw;
    }
    BARK_HIP_CHECK(hipStreamEndCapture(cap_stream, &g));
    const hipError_t e = hipGraphInstantiate(&graph_exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    BARK_HIP_CHECK(e);
    graph_key = key;
    BARK_HIP_CHECK(hipGraphLaunch(graph_exec, st));
  }

  void encode_mel_batch(const float* mel_in, bool mel_on_device, const int32_t* frames,
                        const int32_t* valid, int batch, int32_t* t_out, float* out,
                        bool out_on_device, size_t cap, hipStream_t st,
                        std::vector<std::pair<int, int>>* rows_out = nullptr) {
    BARK_REQUIRE(finalized, "encode before finalize");
    BARK_REQUIRE(batch >= 1 && frames, "batch must be >= 1");
    Plan pl = make_plan(frames, valid, nullptr, batch);
    size_t need_out = 0, total_frames = 0;
    for (const auto& s : pl.seqs) {
      need_out += (size_t)s.t * PROJ;
      total_frames += (size_t)s.frames;
    }
    BARK_REQUIRE(!out || cap >= need_out, "pooler capacity too small");
    ensure_workspace(pl);
    ensure_front_end(pl);
    const float* dmel = mel_in;
    if (!mel_on_device) {
      ensure(mel, total_frames * MEL * 4);
      BARK_HIP_CHECK(hipMemcpyAsync(mel.p, mel_in, total_frames * MEL * 4,
                                    hipMemcpyHostToDevice, st));
      dmel = mel.as<float>();
    }
    upload_tables(pl, st);
    auto body = [&](hipStream_t s_) {
      zero_fill(sub16.p, (size_t)pl.mp * 4096 * 2, s_);
      size_t foff = 0;
      for (const auto& s : pl.seqs) {
        front_end(dmel + foff * MEL, s, s_);
        foff += s.frames;
      }
      encoder_blocks(pl, -1, s_);
    };
    std::vector<long> key{pl.mp, pl.tc, (long)reinterpret_cast<uintptr_t>(dmel), ws_gen};
    for (const auto& s : pl.seqs) key.insert(key.end(), {s.frames, s.valid, s.t, s.start});
    run_graphed(key, body, st);
    size_t orow = 0;
    if (rows_out) rows_out->clear();
    for (size_t i = 0; i < pl.seqs.size(); ++i) {
      const auto& s = pl.seqs[i];
      if (t_out) t_out[i] = s.t;
      if (rows_out) rows_out->push_back({s.start, s.t});
      if (!out) continue;
      const float* src = pooler.as<float>() + (size_t)s.start * PROJ;
      BARK_HIP_CHECK(hipMemcpyAsync(out + orow * PROJ, src, (size_t)s.t * PROJ * 4,
                                    out_on_device ? hipMemcpyDeviceToDevice
                                                  : hipMemcpyDeviceToHost,
                                    st));
      orow += s.t;
    }
    if (out && !out_on_device) BARK_HIP_CHECK(hipStreamSynchronize(st));
  }

  // log-mel of each wave (packed frames), then one batched encode
  void encode_wave_batch(const float* waves, const int64_t* n_samples, int batch, int32_t* t_out, float* out,
                         size_t cap) {
    BARK_REQUIRE(batch >= 1 && waves && n_samples, "batch must be >= 1");
    std::vector<int32_t> frames(batch), valid(batch);
    size_t total_samples = 0, total_frames = 0;
    for (int i = 0; i < batch; ++i) {
      BARK_REQUIRE(n_samples[i] > 0, "empty wave");
      total_samples += (size_t)n_samples[i];
      frames[i] = mel_frames(n_samples[i]);
      total_frames += (size_t)frames[i];
    }
    hipStream_t st = stream;
    ensure(mel_wave, total_samples * 4);
    ensure(mel, total_frames * MEL * 4);
    BARK_HIP_CHECK(hipMemcpyAsync(mel_wave.p, waves, total_samples * 4, hipMemcpyHostToDevice, st));
    size_t soff = 0, foff = 0;
    for (int i = 0; i < batch; ++i) {
      run_mel(mel_wave.as<float>() + soff, (long)n_samples[i], mel.as<float>() + foff * MEL, (size_t)frames[i] * MEL,
              &frames[i], &valid[i], st);
      soff += (size_t)n_samples[i];
      foff += (size_t)frames[i];
    }
    encode_mel_batch(mel.as<float>(), true, frames.data(), valid.data(), batch, t_out, out, false, cap, st);
  }

  // Transcription of a batch of waves up to the tokens (AsrInference's
  // mel -> encoder -> decoder, src/transcription.rs:56-224, chunk by chunk as
  // src/inference.rs:298-386): log-mel of every wave, one batched encode, and
  // a greedy TDT decode of each wave's pooler where the encoder left it; only
  // the tokens leave the device. Wave i's n_tokens[i] {id, frame, dur} triples
  // follow those of the waves before it.
  void transcribe_wave_batch(const float* waves, const int64_t* n_samples, int batch, int32_t* t_out,
                             uint32_t* tokens, size_t cap, int32_t* n_tokens) {
    BARK_REQUIRE(has_tdt, "no TDT decoder tensors were set before finalize");
    BARK_REQUIRE(batch >= 1 && waves && n_samples && n_tokens, "batch must be >= 1");
    std::vector<int32_t> frames(batch), valid(batch);
    size_t total_samples = 0, total_frames = 0;
    for (int i = 0; i < batch; ++i) {
      BARK_REQUIRE(n_samples[i] > 0, "empty wave");
      total_samples += (size_t)n_samples[i];
      frames[i] = mel_frames(n_samples[i]);
      total_frames += (size_t)frames[i];
    }
    hipStream_t st = stream;
    ensure(mel_wave, total_samples * 4);
    ensure(mel, total_frames * MEL * 4);
    BARK_HIP_CHECK(hipMemcpyAsync(mel_wave.p, waves, total_samples * 4, hipMemcpyHostToDevice, st));
    size_t soff = 0, foff = 0;
    for (int i = 0; i < batch; ++i) {
      run_mel(mel_wave.as<float>() + soff, (long)n_samples[i], mel.as<float>() + foff * MEL, (size_t)frames[i] * MEL,
              &frames[i], &valid[i], st);
      soff += (size_t)n_samples[i];
      foff += (size_t)frames[i];
    }
    std::vector<std::pair<int, int>> rows;
    encode_mel_batch(mel.as<float>(), true, frames.data(), valid.data(), batch, t_out, nullptr, true, 0, st, &rows);
    std::vector<int> r0(batch), tl(batch);
    for (int i = 0; i < batch; ++i) {
      r0[i] = rows[i].first;
      tl[i] = rows[i].second;
    }
    tdt_decode_copy(pooler.as<float>(), r0.data(), tl.data(), batch, tokens, cap, n_tokens, st);
  }

  void encode_sub(const float* sub_rows, int t, int dump_layer, float* out_pooler,
                  float* out_block) {
    BARK_REQUIRE(finalized, "encode before finalize");
    BARK_REQUIRE(t >= 1, "t must be >= 1");
    BARK_REQUIRE(dump_layer < n_layers, "dump_layer out of range");
    const int32_t tl = t;
    Plan pl = make_plan(nullptr, nullptr, &tl, 1);
    ensure_workspace(pl);
    ensure(subf32, (size_t)t * 4096 * 4);
    hipStream_t st = stream;
    BARK_HIP_CHECK(hipMemcpyAsync(subf32.p, sub_rows, (size_t)t * 4096 * 4,
                                  hipMemcpyHostToDevice, st));
    upload_tables(pl, st);
    zero_fill(sub16.p, (size_t)pl.mp * 4096 * 2, st);
    f32_to_f16_rows(subf32.as<float>(), t, 4096, sub16.as<half>(), 4096, st);
    encoder_blocks(pl, dump_layer, st);
    if (out_pooler)
      BARK_HIP_CHECK(hipMemcpyAsync(out_pooler, pooler.p, (size_t)t * PROJ * 4,
                                    hipMemcpyDeviceToHost, st));
    if (out_block && dump_layer >= 0)
      BARK_HIP_CHECK(hipMemcpyAsync(out_block, dump.p, (size_t)t * HIDDEN * 4,
                                    hipMemcpyDeviceToHost, st));
    BARK_HIP_CHECK(hipStreamSynchronize(st));
  }
};

// -------------------------------------------------------------------- C ABI --
namespace {

template <class F>
int guarded(F&& f) {
  try {
    f();
    g_last_error.clear();
    return BARK_HIP_OK;
  } catch (const Error& e) {
    g_last_error = e.msg;
    if (e.msg.find("hip") != std::string::npos) return BARK_HIP_EDEVICE;
    if (e.msg.find("before finalize") != std::string::npos ||
        e.msg.find("twice") != std::string::npos)
      return BARK_HIP_ESTATE;
    return BARK_HIP_EINVAL;
  } catch (const std::exception& e) {
    g_last_error = std::string("internal error: ") + e.what();
    return BARK_HIP_EINTERNAL;
  } catch (...) {
    g_last_error = "internal error";
    return BARK_HIP_EINTERNAL;
  }
}

HostTensor& stage(BarkHip* h, const char* name) {
  BARK_REQUIRE(h && name, "null handle or name");
  BARK_REQUIRE(!h->finalized, "tensors cannot be set after finalize");
  return h->staged[name];
}

}  // namespace

namespace {
void lowbit_linear_checked(const void* A, int32_t a_dtype, const uint8_t* codes, const uint16_t* lut16, void* C,
                           int32_t c_dtype, int32_t T, int32_t K, int32_t N, void* stream, bool noalloc) {
  BARK_REQUIRE(A && codes && lut16 && C, "null device pointer");
  BARK_REQUIRE(a_dtype == 0 || a_dtype == 1, "a_dtype must be 0 (f16) or 1 (bf16)");
  BARK_REQUIRE(c_dtype >= 0 && c_dtype <= 2, "c_dtype must be 0, 1 or 2");
  BARK_REQUIRE(T >= 1, "T must be >= 1");
  GemmWeight w;
  w.codes = codes;
  w.lut = reinterpret_cast<const half*>(lut16);
  w.n = N;
  w.k = K;
  BARK_REQUIRE(K % 256 == 0 && K > 0, "K must be a positive multiple of 256");
  BARK_REQUIRE(N % 128 == 0 && N > 0, "N must be a positive multiple of 128");
  if (noalloc)
    gemm_isolated_noalloc(static_cast<const half*>(A), T, w, C, c_dtype, static_cast<hipStream_t>(stream),
                          a_dtype == 1);
  else
    gemm_isolated(static_cast<const half*>(A), T, w, C, c_dtype, static_cast<hipStream_t>(stream), a_dtype == 1);
}
}  // namespace

extern "C" {

const char* bark_hip_last_error(void) { return g_last_error.c_str(); }

int bark_hip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int bark_hip_create(int device, int n_layers, BarkHip** out) {
  return guarded([&] {
    BARK_REQUIRE(out, "null output pointer");
    *out = nullptr;
    BARK_REQUIRE(n_layers >= 1 && n_layers <= 24, "n_layers must be in 1..24");
    int n = 0;
    BARK_HIP_CHECK(hipGetDeviceCount(&n));
    BARK_REQUIRE(device >= 0 && device < n, "no such HIP device");
    BARK_HIP_CHECK(hipSetDevice(device));
    auto* h = new BarkHip();
    h->device = device;
    h->n_layers = n_layers;
    hipError_t e = hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&h->done, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&h->tables_copied, hipEventDisableTiming);
    if (e != hipSuccess) {
      delete h;
      throw Error{std::string("hipStreamCreate/hipEventCreate: ") + hipGetErrorString(e)};
    }
    *out = h;
  });
}

void bark_hip_destroy(BarkHip* h) {
  if (!h) return;
  (void)hipSetDevice(h->device);
  delete h;
}

int bark_hip_set_f32(BarkHip* h, const char* name, const float* v, const int64_t* shape,
                     int ndim) {
  return guarded([&] {
    BARK_REQUIRE(v && shape && ndim >= 1 && ndim <= 8, "bad f32 tensor arguments");
    std::lock_guard<std::mutex> lk(h->mu);
    HostTensor& t = stage(h, name);
    t = HostTensor();
    t.kind = HostTensor::F32;
    t.shape.assign(shape, shape + ndim);
    for (int64_t d : t.shape) BARK_REQUIRE(d >= 0, "negative dimension");
    const int64_t n = shape_elements(t.shape, name ? name : "tensor");
    BARK_REQUIRE(n > 0, "empty tensor");
    t.f32.assign(v, v + n);
  });
}

int bark_hip_set_f16(BarkHip* h, const char* name, const uint16_t* v, int64_t rows,
                     int64_t cols) {
  return guarded([&] {
    BARK_REQUIRE(v && rows > 0 && cols > 0, "bad f16 tensor arguments");
    std::lock_guard<std::mutex> lk(h->mu);
    HostTensor& t = stage(h, name);
    t = HostTensor();
    t.kind = HostTensor::F16;
    t.shape = {rows, cols};
    t.rows = rows;
    t.cols = cols;
    t.f16.assign(v, v + rows * cols);
  });
}

int bark_hip_set_lowbit(BarkHip* h, const char* name, const uint32_t* codes,
                        const uint16_t* levels, uint32_t k_lev, int64_t rows, int64_t cols) {
  return guarded([&] {
    BARK_REQUIRE(codes && levels && rows > 0 && cols > 0, "bad low-bit tensor arguments");
    BARK_REQUIRE(k_lev >= 1 && k_lev <= 3, "unsupported level count (1..3)");
    BARK_REQUIRE(cols % 8 == 0, "low-bit columns must be a multiple of 8");
    std::lock_guard<std::mutex> lk(h->mu);
    HostTensor& t = stage(h, name);
    t = HostTensor();
    t.kind = HostTensor::LUT4;
    t.shape = {rows, cols};
    t.rows = rows;
    t.cols = cols;
    // u32 words with nibble col&7 of word col>>3 are, byte for byte on a
    // little-endian host, two codes per byte with the low nibble first.
    t.codes.resize((size_t)rows * cols / 2);
    std::memcpy(t.codes.data(), codes, t.codes.size());
    t.lut.resize((size_t)rows * 16);
    for (int64_t r = 0; r < rows; ++r)
      for (uint32_t c = 0; c < 16; ++c)
        t.lut[r * 16 + c] = f32_to_f16_bits(expand_level(c, k_lev, levels + r * 4));
  });
}

int bark_hip_set_lut4(BarkHip* h, const char* name, const uint8_t* codes, const uint16_t* lut16,
                      int64_t rows, int64_t cols) {
  return guarded([&] {
    BARK_REQUIRE(codes && lut16 && rows > 0 && cols > 0, "bad 4-bit tensor arguments");
    BARK_REQUIRE(cols % 2 == 0, "4-bit columns must be even");
    std::lock_guard<std::mutex> lk(h->mu);
    HostTensor& t = stage(h, name);
    t = HostTensor();
    t.kind = HostTensor::LUT4;
    t.shape = {rows, cols};
    t.rows = rows;
    t.cols = cols;
    t.codes.assign(codes, codes + rows * cols / 2);
    t.lut.assign(lut16, lut16 + rows * 16);
  });
}

int bark_hip_load_safetensors(BarkHip* h, const char* path) {
  return guarded([&] {
    BARK_REQUIRE(h && path, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_REQUIRE(!h->finalized, "tensors cannot be set after finalize");
    // the tensors this handle reads: front end, encoder blocks below n_layers,
    // projector, TDT decoder and joint
    auto wanted = [&](const std::string& n) {
      const std::string blocks = "encoder.layers.";
      if (n.compare(0, blocks.size(), blocks) == 0) {
        const size_t dot = n.find('.', blocks.size());
        if (dot == std::string::npos) return false;
        const std::string l = n.substr(blocks.size(), dot - blocks.size());
        if (l.empty() || l.size() > 3 || l.find_first_not_of("0123456789") != std::string::npos) return false;
        return std::stoi(l) < h->n_layers;
      }
      for (const char* pre : {"encoder.subsampling.", "encoder_projector.", "decoder.", "joint."})
        if (n.compare(0, std::strlen(pre), pre) == 0) return true;
      return false;
    };
    for (const std::string& file : safetensors_files(path)) {
      for (const StTensor& t : safetensors_header(file)) {
        if (!wanted(t.name)) continue;
        const int64_t n = t.numel;  // overflow-checked by the header reader
        const uint64_t bytes = t.end - t.begin;
        HostTensor v;
        v.shape = t.shape;
        if (t.dtype == "F32") {
          BARK_REQUIRE(bytes == (uint64_t)n * 4, t.name + ": size does not match its shape");
          v.kind = HostTensor::F32;
          v.f32.resize(n);
          safetensors_read(file, t, v.f32.data());
        } else if (t.dtype == "F16") {
          BARK_REQUIRE(bytes == (uint64_t)n * 2, t.name + ": size does not match its shape");
          v.kind = HostTensor::F16;
          v.f16.resize(n);
          safetensors_read(file, t, v.f16.data());
          v.rows = t.shape.empty() ? 1 : t.shape[0];
          v.cols = v.rows ? n / v.rows : 0;
        } else if (t.dtype == "BF16") {  // widened exactly (RawTensor::to_f32, src/raw.rs:23-48)
          BARK_REQUIRE(bytes == (uint64_t)n * 2, t.name + ": size does not match its shape");
          std::vector<uint16_t> raw(n);
          safetensors_read(file, t, raw.data());
          v.kind = HostTensor::F32;
          v.f32.resize(n);
          for (int64_t k = 0; k < n; ++k) {
            const uint32_t u = (uint32_t)raw[k] << 16;
            std::memcpy(&v.f32[k], &u, 4);
          }
        } else {
          continue;  // integer entries (BatchNorm's num_batches_tracked) are never read
        }
        BARK_REQUIRE(n > 0, t.name + ": empty tensor");
        stage(h, t.name.c_str()) = std::move(v);
      }
    }
  });
}

int bark_hip_probe(const char* path, char* buf, size_t cap) {
  return guarded([&] {
    BARK_REQUIRE(path && buf && cap > 0, "null argument");
    const std::string r = safetensors_probe(path);
    BARK_REQUIRE(r.size() < cap, "buffer too small for the probe result");
    std::memcpy(buf, r.c_str(), r.size() + 1);
  });
}

int bark_hip_finalize(BarkHip* h) {
  return guarded([&] {
    BARK_REQUIRE(h, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    h->finalize();
  });
}

int bark_hip_encode_sub(BarkHip* h, const float* sub_rows, int32_t t, int32_t dump_layer,
                        float* pooler, float* block) {
  return guarded([&] {
    BARK_REQUIRE(h && sub_rows, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    h->on_stream(h->stream, [&] { h->encode_sub(sub_rows, t, dump_layer, pooler, block); });
  });
}

int bark_hip_encode_mel(BarkHip* h, const float* mel, int32_t n_frames, int32_t n_valid,
                        int32_t* t_out, float* pooler, size_t pooler_cap) {
  return guarded([&] {
    BARK_REQUIRE(h && mel && pooler, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    h->on_stream(h->stream, [&] {
      h->encode_mel_batch(mel, false, &n_frames, &n_valid, 1, t_out, pooler, false, pooler_cap, h->stream);
    });
  });
}

int bark_hip_encode_mel_batch(BarkHip* h, const float* mel, const int32_t* n_frames,
                              const int32_t* n_valid, int32_t batch, int32_t* t_out,
                              float* pooler, size_t pooler_cap) {
  return guarded([&] {
    BARK_REQUIRE(h && mel && pooler, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    h->on_stream(h->stream, [&] {
      h->encode_mel_batch(mel, false, n_frames, n_valid, batch, t_out, pooler, false, pooler_cap, h->stream);
    });
  });
}

int bark_hip_encode_mel_batch_device(BarkHip* h, const float* d_mel, const int32_t* n_frames,
                                     const int32_t* n_valid, int32_t batch, int32_t* t_out,
                                     float* d_pooler, size_t pooler_cap, void* stream) {
  return guarded([&] {
    BARK_REQUIRE(h && d_mel && d_pooler, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    hipStream_t st = stream ? static_cast<hipStream_t>(stream) : h->stream;
    h->on_stream(st, [&] {
      h->encode_mel_batch(d_mel, true, n_frames, n_valid, batch, t_out, d_pooler, true, pooler_cap, st);
    });
  });
}

int bark_hip_set_mel_filters(BarkHip* h, const float* filters) {
  return guarded([&] {
    BARK_REQUIRE(h && filters, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    h->set_mel_filters(filters);
  });
}

int bark_hip_mel(BarkHip* h, const float* wave, int64_t n_samples, float* features, size_t cap, int32_t* n_frames,
                 int32_t* n_valid) {
  return guarded([&] {
    BARK_REQUIRE(h && wave && features, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    BARK_REQUIRE(n_samples > 0, "empty wave");
    const size_t nf = (size_t)mel_frames(n_samples);
    BARK_REQUIRE(cap >= nf * MEL, "features buffer too small");
    h->ensure(h->mel_wave, (size_t)n_samples * 4);
    h->ensure(h->mel_feat, nf * MEL * 4);
    h->on_stream(h->stream, [&] {
      BARK_HIP_CHECK(hipMemcpyAsync(h->mel_wave.p, wave, (size_t)n_samples * 4, hipMemcpyHostToDevice, h->stream));
      h->run_mel(h->mel_wave.as<float>(), (long)n_samples, h->mel_feat.as<float>(), nf * MEL, n_frames, n_valid,
                 h->stream);
      BARK_HIP_CHECK(hipMemcpyAsync(features, h->mel_feat.p, nf * MEL * 4, hipMemcpyDeviceToHost, h->stream));
      BARK_HIP_CHECK(hipStreamSynchronize(h->stream));
    });
  });
}

int bark_hip_mel_device(BarkHip* h, const float* d_wave, int64_t n_samples, float* d_features, size_t cap,
                        int32_t* n_frames, int32_t* n_valid, void* stream) {
  return guarded([&] {
    BARK_REQUIRE(h && d_wave && d_features, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    hipStream_t st = stream ? static_cast<hipStream_t>(stream) : h->stream;
    h->on_stream(st, [&] { h->run_mel(d_wave, (long)n_samples, d_features, cap, n_frames, n_valid, st); });
  });
}

int bark_hip_encode_wave_batch(BarkHip* h, const float* waves, const int64_t* n_samples, int32_t batch,
                               int32_t* t_out, float* pooler, size_t pooler_cap) {
  return guarded([&] {
    BARK_REQUIRE(h && waves && n_samples && pooler, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    h->on_stream(h->stream, [&] { h->encode_wave_batch(waves, n_samples, batch, t_out, pooler, pooler_cap); });
  });
}

int bark_hip_tdt_decode(BarkHip* h, const float* pooler, int32_t t_len, uint32_t* tokens, size_t cap,
                        int32_t* n_tokens) {
  return bark_hip_tdt_decode_batch(h, pooler, &t_len, 1, tokens, cap, n_tokens);
}

int bark_hip_tdt_decode_device(BarkHip* h, const float* d_pooler, int32_t t_len, uint32_t* tokens, size_t cap,
                               int32_t* n_tokens, void* stream) {
  return bark_hip_tdt_decode_batch_device(h, d_pooler, &t_len, 1, tokens, cap, n_tokens, stream);
}

int bark_hip_tdt_decode_batch(BarkHip* h, const float* pooler, const int32_t* t_lens, int32_t batch, uint32_t* tokens,
                              size_t cap, int32_t* n_tokens) {
  return guarded([&] {
    BARK_REQUIRE(h && t_lens && batch >= 1, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    std::vector<int> rows(batch);
    size_t total = 0;
    for (int u = 0; u < batch; ++u) {
      BARK_REQUIRE(t_lens[u] >= 0 && t_lens[u] <= (1 << 24), "t_len out of range");
      rows[u] = (int)total;
      total += (size_t)t_lens[u];
      BARK_REQUIRE(total < (1u << 31), "too many frames");
    }
    BARK_REQUIRE(pooler || total == 0, "null pooler");
    if (total > 0) h->ensure(h->tdt_pooler, total * 640 * 4);
    h->on_stream(h->stream, [&] {
      if (total > 0)
        BARK_HIP_CHECK(hipMemcpyAsync(h->tdt_pooler.p, pooler, total * 640 * 4, hipMemcpyHostToDevice, h->stream));
      h->tdt_decode_copy(h->tdt_pooler.as<float>(), rows.data(), t_lens, batch, tokens, cap, n_tokens, h->stream);
    });
  });
}

int bark_hip_tdt_decode_batch_device(BarkHip* h, const float* d_pooler, const int32_t* t_lens, int32_t batch,
                                     uint32_t* tokens, size_t cap, int32_t* n_tokens, void* stream) {
  return guarded([&] {
    BARK_REQUIRE(h && t_lens && batch >= 1, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    hipStream_t st = stream ? static_cast<hipStream_t>(stream) : h->stream;
    std::vector<int> rows(batch);
    size_t total = 0;
    for (int u = 0; u < batch; ++u) {
      BARK_REQUIRE(t_lens[u] >= 0 && t_lens[u] <= (1 << 24), "t_len out of range");
      rows[u] = (int)total;
      total += (size_t)t_lens[u];
      BARK_REQUIRE(total < (1u << 31), "too many frames");
    }
    h->on_stream(st, [&] { h->tdt_decode_copy(d_pooler, rows.data(), t_lens, batch, tokens, cap, n_tokens, st); });
  });
}

int bark_hip_transcribe_wave_batch(BarkHip* h, const float* waves, const int64_t* n_samples, int32_t batch,
                                   int32_t* t_out, uint32_t* tokens, size_t cap, int32_t* n_tokens) {
  return guarded([&] {
    BARK_REQUIRE(h && waves && n_samples && n_tokens, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    h->on_stream(h->stream, [&] { h->transcribe_wave_batch(waves, n_samples, batch, t_out, tokens, cap, n_tokens); });
  });
}

int bark_hip_profile(BarkHip* h, int enable) {
  return guarded([&] {
    BARK_REQUIRE(h, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    (void)h->prof.report();  // drop anything recorded so far
    h->prof.on = enable != 0;
  });
}

int bark_hip_profile_only(BarkHip* h, const char* label) {
  return guarded([&] {
    BARK_REQUIRE(h, "null handle");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    (void)h->prof.report();
    h->prof.only = label ? label : "";
    h->prof.only_seen = 0;
  });
}

int bark_hip_profile_report(BarkHip* h, char* buf, size_t cap) {
  return guarded([&] {
    BARK_REQUIRE(h && buf && cap > 0, "null argument");
    std::lock_guard<std::mutex> lk(h->mu);
    BARK_HIP_CHECK(hipSetDevice(h->device));
    const std::string r = h->prof.report();
    BARK_REQUIRE(r.size() + 1 <= cap, "profile report buffer too small");
    std::memcpy(buf, r.c_str(), r.size() + 1);
  });
}


int bark_hip_lowbit_linear_noalloc(const void* A, int32_t a_dtype, const uint8_t* codes, const uint16_t* lut16,
                                   void* C, int32_t c_dtype, int32_t T, int32_t K, int32_t N, void* stream) {
  return guarded([&] { lowbit_linear_checked(A, a_dtype, codes, lut16, C, c_dtype, T, K, N, stream, true); });
}

int bark_hip_lowbit_linear(const void* A, int32_t a_dtype, const uint8_t* codes,
                           const uint16_t* lut16, void* C, int32_t c_dtype, int32_t T,
                           int32_t K, int32_t N, void* stream) {
  return guarded([&] { lowbit_linear_checked(A, a_dtype, codes, lut16, C, c_dtype, T, K, N, stream, false); });
}

}  // extern "C"
