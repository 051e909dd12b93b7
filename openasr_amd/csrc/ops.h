// ops.h -- host-side launchers of the gfx950 kernels. Every launcher only
// enqueues work on the given stream; shapes are validated by the planner
// (mi355x_exec.cpp) before a launcher is reached.
#pragma once

#include "mi355x_common.h"

namespace mi355x {

struct act_buffers {
    int8_t * q;
    float * d;
    int16_t * ssum;  // Q8_K only: sums of each 32 consecutive quants, [col][K/32]
};

// activation quantization for a quantized-weight MUL_MAT
void launch_quantize_act(const tview & src, int wtype, const act_buffers & out, hipStream_t stream);
size_t act_bytes(int wtype, int64_t K, int64_t ncols);
act_buffers act_carve(int wtype, char * base, int64_t K, int64_t ncols);

// GEMV on Q8_0 (row-split) / Q4_K / Q3_K weights for N columns, dst column stride dst_nb1 bytes
void launch_mmv(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                int64_t N, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu);

// Activation prologue of the MFMA GEMV: instead of reading pre-quantized
// activations, every workgroup reads the f32 activations x (column stride
// x_nb1 bytes), optionally normalises each column (RMS_NORM or NORM, then
// * w, + b -- the ops the graph applies before the MUL_MAT) and quantizes
// them into LDS with the same arithmetic as the stand-alone norm and
// quantize kernels.
struct gemv_prologue {
    const float * x = nullptr;
    int64_t x_nb1 = 0;
    const float * w = nullptr;
    const float * b = nullptr;
    float eps = 0.0f;
    int norm = -1;  // -1: quantize only; 0: RMS norm; 1: layer norm
};

// MFMA GEMV for the decode step (16-column chunks), M % 16 == 0; res (same
// column layout as dst, stride res_nb1) is added to the result when non-null;
// with W2 (same shape and type as W) the result is silu(W x) * (W2 x). With a
// prologue, act is not read.
bool gemv_mfma_supported(int wtype, int64_t M, int64_t K);
// whether a launch of this shape can take the activation prologue
bool gemv_prologue_supported(int wtype, int64_t M, int64_t K, int64_t N, bool norm);
// Further epilogue of a one-column Q8_0 launch (the single-column form),
// after the residual: a second addend of the output's shape (the bias, then
// the residual: two roundings as the unfused ADDs), or GELU through ggml's f16
// table.
// the single-column form takes a launch of one column of Q8_0 weights (K
// within its passes; with a normalising prologue, K within its waves' groups)
bool gemv_single_column(int wtype, int64_t K, int64_t N, bool norm);

struct gemv_epilogue {
    const char * res2 = nullptr;
    const uint16_t * gelu = nullptr;
};

// Further matrices of a one-column launch with a normalising prologue: sibling
// MUL_MATs of the same normalised input (Whisper's q, k, v projections), each
// with its own rows, output and optional residual (a folded bias).
struct gemv_sub {
    const char * W = nullptr;
    int64_t M = 0;
    char * dst = nullptr;
    const char * res = nullptr;
    // optional SET_ROWS of the result column into an f16 cache: element m
    // to rows_dst + r * rows_nb1 + 2 m with r = rows_idx[0] (I32, or I64 when
    // rows_i64), skipped unless 0 <= r < rows_n (Whisper's self-attention K / V)
    char * rows_dst = nullptr;
    const char * rows_idx = nullptr;
    int rows_i64 = 0;
    int64_t rows_nb1 = 0, rows_n = 0;
};
constexpr int kGemvMaxSubs = 2;

void launch_gemv_mfma(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                      int64_t N, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu,
                      const char * res = nullptr, int64_t res_nb1 = 0, const char * W2 = nullptr,
                      const gemv_prologue * pro = nullptr, const gemv_epilogue & epi = gemv_epilogue(),
                      const gemv_sub * subs = nullptr, int nsub = 0);

// MFMA int8 GEMM for wider N (prefill)
bool mmq_supported(int wtype, int64_t M, int64_t K);
struct gemm_float_epi;
struct gemm_float_sub;
// subs: sibling products of the same activations in one launch (weights of
// the same type, K and row stride; contiguous outputs of N columns; each
// product's rows a multiple of 64; only a bias in the epilogue)
void launch_mmq(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                int64_t N, char * dst, int64_t dst_nb1, hipStream_t stream, int n_cu, const gemm_float_epi & epi,
                const gemm_float_sub * subs = nullptr, int nsub = 0);

// the same product at the default precision on the f16 matrix cores
// (k_mmq_f16.hip, float tolerance): where it takes the product (enough
// 128 x 128 tiles), the general scratch it needs (the activations
// dequantized to f16), and the launch (subs joined when every product's rows
// are a multiple of 128)
bool mmq_f16_supported(int wtype, int64_t M, int64_t K, int64_t N, int n_cu);
size_t mmq_f16_scratch_bytes(int64_t K, int64_t N);
// W2: the SwiGLU pair -- dst = silu(W x) * (W2 x), W2 of W's shape, M a
// multiple of 64, no epilogue adds and no subs
void launch_mmq_f16(int wtype, const char * W, int64_t row_bytes, int64_t M, int64_t K, const act_buffers & act,
                    int64_t N, char * dst, int64_t dst_nb1, void * scratch, hipStream_t stream,
                    const gemm_float_epi & epi, const gemm_float_sub * subs = nullptr, int nsub = 0,
                    const char * W2 = nullptr);

// float GEMM fallback (f16 / f32 src0)
void launch_mul_mat_float(const tview & d, const tview & a, int atype, const tview & b, hipStream_t s);

// float-weight MUL_MAT on the matrix cores (k_gemm_float.hip): src0 a (F16 /
// F32, rows contiguous) x src1 b (F32 / F16, rows contiguous) -> d (f32),
// batch dims broadcast from a as ggml does (r2 = d.ne2 / a.ne2, r3)
// optional epilogue: out = (acc + bias[row]) + res[row, col] (res laid out as
// the output), then GELU_ERF -- the roundings of MUL_MAT, ADD, ADD, GELU_ERF
// apart. A convolution's column GEMM (k_gemm_float only) may instead add a
// bias of one value a column (bias_col) and write its permuted layout: with
// perm_rows = P, row m and column n go to element (m % P) + P n + P N (m / P)
// of a contiguous output (ggml_conv_2d's PERMUTE(0, 1, 3, 2) + CONT)
struct gemm_float_epi {
    const float * bias = nullptr;
    const float * res = nullptr;
    bool gelu_erf = false;
    const float * bias_col = nullptr;
    int64_t perm_rows = 0;
};
constexpr int kGemmFloatMaxSubs = 2;
struct gemm_float_args {
    gemm_float_epi epi;
    const char * a;
    int64_t a_nb1, a_nb2, a_nb3;
    const char * b;
    int64_t b_nb1, b_nb2, b_nb3;
    char * d;
    int64_t d_nb1, d_nb2, d_nb3;
    int64_t M, N, K;
    int ne2, ne3, r2, r3;
    int a_f16, b_f16, a_vec, b_vec;
    // the bf16 form's tile order: workgroup i (of the x dim) on XCD i % 8
    // takes tile (i % 8) per_xcd + i / 8 (none from tiles on), tile t = row
    // tile t / col_blocks, column tile t % col_blocks
    int64_t tiles, col_blocks, per_xcd;
    // split K: workgroup z = s sums k in [s k_span, (s + 1) k_span) into
    // part + s M N (column-major M x N f32), a second launch adds the splits
    // in order and applies the epilogue
    int splits;
    int64_t k_span;
    float * part;
    // sibling products of the same columns in one launch (aligned form, no
    // split): rows [sub_m0[i], sub_m0[i + 1]) of the launch are product i,
    // with weights sub_a[i], contiguous output sub_d[i] and bias sub_bias[i]
    // (product 0 is a / d / epi.bias); every sub_m0 is a multiple of 64
    int nsub;
    int64_t sub_m0[kGemmFloatMaxSubs + 2];
    const char * sub_a[kGemmFloatMaxSubs + 1];
    char * sub_d[kGemmFloatMaxSubs + 1];
    const float * sub_bias[kGemmFloatMaxSubs + 1];
};
// a further product of a sibling launch: weights a (same type, K and row
// stride as the first), output d (f32, contiguous, the first's column count),
// optional bias of one value a row
struct gemm_float_sub {
    const char * a = nullptr;
    int64_t M = 0;
    char * d = nullptr;
    const float * bias = nullptr;
};
bool gemm_float_supported(const tview & d, const tview & a, int atype, const tview & b, int btype);
// how many K splits a launch of this product takes on n_cu CUs (1: none;
// more when its 64 x 64 tiles leave CUs idle), and the f32 partials scratch
// they need
int gemm_float_splits(const tview & d, const tview & a, int atype, const tview & b, int btype, int n_cu);
size_t gemm_float_split_bytes(const tview & d, int splits);
// x3: an F32 x F32 product at the default precision (the graph's contract,
// float tolerance) on the bf16 matrix cores -- each f32 operand element split
// into bf16 hi + lo, three bf16 products a term (hi hi + hi lo + lo hi,
// ~1e-5 relative) -- where the aligned form runs it; else f32 products.
// a_split: src0 holds the split layout IM2COL writes (im2col_args::split);
// only the aligned x3 form reads it, any other launch fails
void launch_gemm_float(const tview & d, const tview & a, int atype, const tview & b, int btype, hipStream_t s,
                       const gemm_float_epi & epi = gemm_float_epi(), int splits = 1, float * part = nullptr,
                       const gemm_float_sub * subs = nullptr, int nsub = 0, bool x3 = false,
                       bool a_split = false);
// whether launch_gemm_float runs this F32 x F32 product in the aligned bf16
// form (x3), the one that reads an a_split operand
bool gemm_float_x3_aligned(const tview & a, const tview & b);
// whether sibling products can join a launch of this product (aligned rows,
// K % 8 == 0, one batch, M a multiple of 64)
bool gemm_float_siblings_ok(const tview & d, const tview & a, const tview & b);

struct fattn_args {
    const char * q;
    const char * k;
    const char * v;
    const char * mask;
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    int64_t m_nb1, m_nb2, m_nb3;
    int m_ne2, m_ne3;
    int d, hq, hkv, n_q, n_kv, n_seq, rk3;
    float scale;
    // launch plan (fattn_plan)
    int tq;        // query positions per tile
    int rows;      // tile rows = tq * (hq / hkv)
    int q_tiles;
    int n_chunks;  // 64-position KV chunks
    int split;     // 0: one workgroup per tile; 1: chunks over workgroups; 2: one wave per chunk
                   // (1 and 2 write partials that a combine launch reduces)
    int dheads;    // split 2: query heads per decode wave (1, or 2 sharing each K/V read)
    // optional quantization of the output for the consuming MUL_MAT:
    // -1 none, GGML_TYPE_Q8_0 or GGML_TYPE_Q4_K (Q8_K activations)
    int qtype;
    act_buffers act;
    // more than one query at the default precision: the matrix-core form
    // (k_fattn_mfma.hip, float tolerance) instead of the chunked definition
    int mfma;
    int mfma_split;  // KV splits of the matrix-core form (partials + combine when > 1)
    // one query at the default precision: the workgroup form (k_fattn_dec.hip,
    // float tolerance); its KV splits (0: not used; > 1: partials + combine)
    int dec;
};
// whether the matrix-core form takes this attention (n_q > 1, D 64 / 128)
bool fattn_mfma_supported(const fattn_args & a);
void fattn_mfma_plan(fattn_args & a, int n_cu);
size_t fattn_mfma_scratch_bytes(const fattn_args & a);
void launch_fattn_mfma(const fattn_args & a, void * scratch, float * out, hipStream_t s);
struct attn_step_args;
// whether the single-query workgroup form takes this attention (n_q = 1,
// D 64 / 128, 1, 2 or 4 query heads a kv head)
bool fattn_dec_supported(const fattn_args & a);
// a.dec: the KV splits where the workgroup form is the faster one, else 0
void fattn_dec_plan(fattn_args & a, int n_cu);
size_t fattn_dec_scratch_bytes(const fattn_args & a);
// step: the fused decode step (st's QK-norm, RoPE, new K / V rows and cache
// writes; D 128); otherwise a plain FLASH_ATTN_EXT over st.fa into out
void launch_fattn_dec(const attn_step_args & st, bool step, float * out, void * scratch, hipStream_t s);
// the combine launch of the split forms over partials laid out per (tile
// row, partial) -- a.n_chunks partials a row, a.rows rows a tile
void launch_fattn_combine(const fattn_args & a, const float * pm, const float * pl, const float * pa, float * out,
                          hipStream_t s);
// The unfused attention chain of the discrete-GPU prefill (MUL_MAT(K, Q) ->
// SOFT_MAX_EXT -> MUL_MAT(CONT(V^T), P) -> PERMUTE/CONT) as one launch, in
// the fixed order k_attn_naive.hip defines. Q f32 [d, n_q, hq, n_seq]
// (strided), K / V f16 [d, n_kv, hkv, n_seq / rk3] rows (16-byte aligned),
// mask f16 [>= n_kv, >= n_q, m_ne2, m_ne3] or null; out f32 [d, hq, n_q,
// n_seq] contiguous. q_f32 / p_f32: GGML_PREC_F32 on the score / context
// product (the operand stays f32), else it is rounded to f16.
constexpr int kNaMaxChunks = 128;  // spans of up to 8192 positions
struct naive_attn_args {
    const char * q;
    const char * k;
    const char * v;
    const char * mask;
    int64_t q_nb1, q_nb2, q_nb3;
    int64_t k_nb1, k_nb2, k_nb3;
    int64_t v_nb1, v_nb2, v_nb3;
    int64_t m_nb1, m_nb2, m_nb3;
    int m_ne2, m_ne3;
    int d, hq, hkv, n_q, n_kv, n_seq, rk3;
    float scale;
    int q_f32, p_f32;
    float * out;
    // set by the launcher
    int qt;        // queries a workgroup owns (16 / (hq / hkv))
    float * work;  // per workgroup 16 rows x the span rounded to 64, f32
};
bool attn_naive_supported(int d, int hq, int hkv, int64_t n_kv);
size_t attn_naive_scratch_bytes(const naive_attn_args & a);
void launch_attn_naive(const naive_attn_args & a, float * work, hipStream_t s);

// REPEAT: dst [ne] filled from src with every index taken modulo src's
// extent in that dim (elements of esize bytes)
void launch_repeat(const tview & d, const tview & src, int esize, hipStream_t s, int n_cu);

// One decode step of attention (D = 128): per-head RMS norm * w and NEOX
// RoPE of the step's new query and key rows (taken from the fused QKV
// projection), the new K/V rows written into the f16 caches at the set_rows
// index, and attention over the cached span by 64-position chunks (the
// flash_attn_ext definition: chunk launch + combine launch). Output: the
// attention rows (and optionally their quantized activations for the output
// projection, fa.qtype / fa.act).
struct attn_step_args {
    fattn_args fa;  // cache reads (k, v, strides), mask, scale, shapes; fa.q unused
    const char * qsrc;  // new query row of head h, sequence s: qsrc + h * q_nb1 + s * q_nb2 (f32)
    int64_t q_nb1, q_nb2;
    const char * ksrc;
    int64_t k_nb1, k_nb2;
    const char * vsrc;
    int64_t v_nb1, v_nb2;
    const float * qw;  // QK-norm weights [128]
    const float * kw;
    float q_eps, k_eps;
    const int32_t * pos;  // RoPE position of sequence s: pos[s]
    float theta_scale, freq_scale, attn_factor;
    const char * idx;  // set_rows index: row of (head h, sequence s) = idx[0, h % ne1, s % ne2]
    int64_t idx_nb1, idx_nb2;
    int idx_ne1, idx_ne2, idx_i64;
    char * kc;  // K / V caches written (f16), [128, rows, hkv, n_seq] strides
    int64_t kc_nb1, kc_nb2, kc_nb3, kc_rows;
    char * vc;
    int64_t vc_nb1, vc_nb2, vc_nb3, vc_rows;
    float * out;  // [128, hq, 1, n_seq]
    const float2 * rope;  // per sequence the 64 (cos, sin) pairs of its position (launch_rope_table)
};
// (cos, sin) of the NEOX rotation angles of 128-wide rows at each sequence's
// position: table[s][i] for rotation index i < 64, the arithmetic of
// k_rms_norm_rope128 (theta_i = p * theta_scale^i built by repeated
// multiplication, deterministic sincos, times attn_factor)
void launch_rope_table(float2 * table, const int32_t * pos, int n_seq, float theta_scale, float freq_scale,
                       float attn_factor, hipStream_t s);
bool attn_step_supported(const fattn_args & a);
size_t attn_step_scratch_bytes(const fattn_args & a);
void launch_attn_step(const attn_step_args & a, void * scratch, hipStream_t stream);

bool fattn_supported(int d, int hq, int hkv);
void fattn_plan(fattn_args & a, int n_cu);
bool fattn_fits(const fattn_args & a);
size_t fattn_scratch_bytes(const fattn_args & a);
void launch_fattn(const fattn_args & a, void * scratch, float * out, hipStream_t stream);

void launch_binary(int op, const tview & d, const tview & a, const tview & b, hipStream_t s, int n_cu);
void launch_scale(const tview & d, const tview & a, float sc, float bias, hipStream_t s, int n_cu);
// launch_unary codes past ggml's unary ops: GGML_OP_SIN / GGML_OP_COS
// (sincosf_det, the deterministic sine and cosine the CPU reference runs)
constexpr int kUnarySin = 1001, kUnaryCos = 1002;
void launch_concat(const tview & d, const tview & a, const tview & b, int dim, int esize, hipStream_t s, int n_cu);
void launch_unary(const tview & d, const tview & a, int op, const uint16_t * gelu_table, hipStream_t s, int n_cu);
void launch_silu_mul(const tview & d, const tview & g, const tview & u, hipStream_t s, int n_cu);
// qtype/act: optionally also write the normalised rows as quantized
// activations (rows = columns of the consuming MUL_MAT); honoured when
// norm_rows_supported() holds, else the caller quantizes separately
void launch_norm(const tview & d, const tview & a, int mode, float eps, const tview * w, const tview * b,
                 hipStream_t s, int qtype = -1, const act_buffers * act = nullptr);
bool norm_rows_supported(const tview & d, const tview & a, const tview * w, const tview * b);
void launch_rope(const tview & d, const tview & a, const int32_t * pos, int n_dims, int mode, float freq_base,
                 float freq_scale, float attn_factor, hipStream_t s, int n_cu);
// optional second job (dst2/src2, same indices): both writes in one launch
void launch_set_rows(const tview & dst, int dtype, const tview & src, const tview & idx, int idx_is_i64,
                     hipStream_t s, int n_cu, const tview * dst2 = nullptr, int dtype2 = 0,
                     const tview * src2 = nullptr);
// RMSNorm * w then RoPE NEOX on rows of exactly 128 elements (n_dims 128);
// an optional second job (the key rows after the query rows) shares the launch
struct norm_rope_job {
    tview d, a;
    const float * w;
    const int32_t * pos;
    float eps, theta_scale, freq_scale, attn_factor;
    int64_t rows;
};
norm_rope_job make_norm_rope_job(const tview & d, const tview & a, float eps, const float * w, const int32_t * pos,
                                 float freq_base, float freq_scale, float attn_factor);
void launch_rms_norm_rope128(const norm_rope_job & j0, const norm_rope_job * j1, hipStream_t s);
void launch_get_rows(const tview & dst, const tview & src, int stype, const tview & idx, hipStream_t s, int n_cu);
void launch_copy(const tview & d, int dtype, const tview & a, int atype, hipStream_t s, int n_cu);
// two copies of equal element count (same types) in one launch
void launch_copy_pair(const tview & d0, const tview & a0, const tview & d1, const tview & a1, int dtype, int atype,
                      hipStream_t s, int n_cu);
void launch_soft_max(const tview & d, const tview & a, const tview * mask, float scale, hipStream_t s);
size_t argmax_scratch_bytes(int64_t ne0, int64_t rows);
void launch_argmax(const tview & a, int32_t * out, int first, void * scratch, hipStream_t s);

// GGML_OP_IM2COL over a contiguous result [K = IC*KH*KW, OW, OH, N] (1-D: KH =
// OH = 1). Input element (n, ic, ih, iw) is f32 at n*nb_n + ic*nb_c + ih*nb_h +
// 4*iw bytes.
struct im2col_args {
    int64_t total, K, OW, OH, IW, IH, nb_n, nb_c, nb_h;
    int KW, KH, s0, s1, p0, p1, d0, d1;
    // f32 dst only, K % 8 == 0: each 8-element group of a row written as its
    // 8 bf16 hi halves then 8 lo halves (x = hi + lo + ~2^-17 x; 32 bytes, the
    // group's f32 size) -- the operand layout of the column GEMM's bf16 form
    // (launch_gemm_float, a_split), its only reader
    int split;
};
void launch_im2col(void * dst, int dst_f16, const char * src, const im2col_args & a, hipStream_t s);
bool norm_supported(int64_t ne0);
// a one-wave kernel that returns after `us` microseconds of device wall clock
void launch_spin_us(double us, int wall_clock_khz, hipStream_t s);

// Staged host uploads: small tensor writes are copied into pinned host
// memory and applied on the device in one launch when the device is next
// used (entry i: bytes [off, off + n) of the pinned area to dst)
struct upload_entry {
    char * dst;
    uint32_t off, n;
};
constexpr int kUploadBatch = 16;  // entries per apply launch
struct upload_batch {
    const char * src;  // the pinned area (device-accessible host memory)
    int n;
    upload_entry e[kUploadBatch];
};
void launch_apply_uploads(const upload_batch & b, hipStream_t s);

// Q8_0 layout conversion between ggml's interleaved blocks and the row-split
// device layout (host side, used by set/get_tensor)
void q8_0_to_split_rows(const uint8_t * src, uint8_t * dst, int64_t rows, int64_t k);
void q8_0_from_split_rows(const uint8_t * src, uint8_t * dst, int64_t rows, int64_t k);

}  // namespace mi355x
