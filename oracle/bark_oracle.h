/*
 * CPU oracle for the Conformer encoder hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A C restatement of the reference CPU backend (BARK3_CPU_ENC=1):
 *   src/cpu/{mod,layer,ops,gemm}.rs, src/sub.rs, src/bark.rs:expand,
 *   src/encoder.rs:pos_embed_f32, src/raw.rs f32<->f16 conversions.
 * It follows the reference's op order and rounding points exactly:
 *   - every GEMM element is one FMA chain over ascending k starting at 0
 *     (src/cpu/gemm.rs:654-671), except the split-k AV product whose partition
 *     depends on a worker count that is an explicit argument here
 *     (src/cpu/gemm.rs:348-415);
 *   - weights are rounded through f16 (`f16v`, src/cpu/mod.rs:33-37);
 *   - K, V and relK are rounded through f16 (src/cpu/ops.rs:258-259,
 *     src/cpu/layer.rs:234-247);
 *   - LayerNorm / softmax reduce in the reference's 256-lane + tree order.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or the timed CPU baseline. The
 * HIP product path never calls it.
 */
#ifndef BARK_ORACLE_H
#define BARK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- conversions (src/raw.rs:118-133, src/cpu/gemm.rs:212-214) ---- */
uint16_t bo_f32_to_f16(float v);
float bo_f16_to_f32(uint16_t h);
uint16_t bo_f32_to_bf16(float v);
float bo_bf16_to_f32(uint16_t b);
void bo_round_f16_array(const float *in, float *out, size_t n);
void bo_f32_to_f16_array(const float *in, uint16_t *out, size_t n);

/* ---- low-bit weights (src/bark.rs:31-48,352-358,597-611) ---- */
float bo_expand(uint32_t code, uint32_t k, const uint16_t *levels);
/* reference LowBitTensor (u32 words, nibble col&7 of word col>>3) -> f32 */
void bo_lowbit_expand(const uint32_t *codes, const uint16_t *levels, uint32_t k,
                      int64_t rows, int64_t cols, float *out);
/* generic per-row 16-entry f16 table, codes two per byte, low nibble = even col */
void bo_lut4_expand(const uint8_t *codes, const uint16_t *lut16, int64_t rows,
                    int64_t cols, float *out);

/* ---- position table (src/encoder.rs:228-245) ---- */
void bo_pos_embed(int t, float *out /* (2t-1) x 1024 */);

/* ---- GEMM (src/cpu/gemm.rs) ---- */
typedef struct bo_packw bo_packw;
bo_packw *bo_pack_rows(const float *w, int n, int k, int half);
void bo_packw_free(bo_packw *w);
void bo_gemm(const float *a, const bo_packw *w, float *c, int m, int n0, int ncols,
             int threads);
void bo_gemm_split_k(const float *a, const bo_packw *w, float *c, int m, int n0,
                     int ncols, int workers, int threads);
/* plain loops for checking the blocked kernel */
void bo_gemm_fma_chain(const float *a, const float *w, float *c, int m, int n, int k);
void bo_gemm_naive_f64(const float *a, const float *w, double *c, int m, int n, int k);

/* ---- elementwise ops (src/cpu/ops.rs) ---- */
void bo_layer_norm(const float *src, float *dst, const float *w, const float *b,
                   int rows, int dim);
void bo_silu(float *x, size_t n);
void bo_glu(const float *src, float *dst, int rows, int c);
void bo_add_scaled(float *a, const float *b, float scale, size_t n);
void bo_add_bias(float *x, const float *bias, int rows, int dim);
void bo_rel_softmax_rows(float *probs, const float *bd, int win, int rows, int t,
                         int q0, int j0, float scale);
void bo_dwconv_bn_silu(const float *src, const float *dw, const float *bn_a,
                       const float *bn_b, float *dst, int rows, int dim);

/* ---- encoder (src/cpu/mod.rs, src/cpu/layer.rs) ---- */
typedef struct bo_encoder bo_encoder;
bo_encoder *bo_encoder_new(int n_layers);
void bo_encoder_free(bo_encoder *e);
/* `name` is a reference tensor name; `v` holds the checkpoint values widened to
 * f32. Returns 0, or -1 for an unknown name / wrong size. */
int bo_encoder_set(bo_encoder *e, const char *name, const float *v, int64_t n);
/* f16 rounding, packing, qkv fusion and BN folding (src/cpu/mod.rs:47-152). */
int bo_encoder_finalize(bo_encoder *e);
/* sub (t, 4096) -> pooler (t, 640) when layers == n_layers, else the pre-norm
 * residual (t, 1024) of block `layers-1` (src/cpu/mod.rs:156-188). */
int bo_encoder_encode(bo_encoder *e, const float *sub, int t, int layers, float *out,
                      int threads, int av_workers);
/* Full encode that also records every block's pre-norm residual:
 * dumps (n_layers, t, 1024), pooler (t, 640). */
int bo_encoder_encode_dump(bo_encoder *e, const float *sub, int t, float *dumps,
                           float *pooler, int threads, int av_workers);
/* One block on x (t,1024) in place, then x <- norm_out(x) if apply_norm_out. */
int bo_encoder_block(bo_encoder *e, int layer, float *x, int t, int apply_norm_out,
                     int threads, int av_workers);

/* ---- conv subsampling (src/sub.rs:11-300) ---- */
int bo_conv_len(int l);
/* weights: l0 (256,9)+256, l2 (256,9)+256, l3 (256,256)+256, l5 (256,9)+256,
 * l6 (256,256)+256; out (T, 4096) with T = conv_len^3(frames). */
int bo_subsample(const float *l0w, const float *l0b, const float *l2w, const float *l2b,
                 const float *l3w, const float *l3b, const float *l5w, const float *l5b,
                 const float *l6w, const float *l6b, const float *mel, int frames,
                 int n_valid, float *out, int threads);

#ifdef __cplusplus
}
#endif
#endif
