/*
 * ggml_host.h -- the ggml-base entry points the OpenASR Rust host binds
 * (crates/openasr-core/src/ggml_runtime/ffi.rs:399-1057), restricted to what
 * the quantized decoder path uses. This build ships its own implementation
 * of them (libggml-base.so, under openasr_amd/host/) because the fork's
 * ggml-base is not vendored; a device plugin imports these symbols exactly as
 * a ggml-hip plugin imports ggml-base.
 *
 * Signatures and argument meaning follow ffi.rs line by line; each group
 * cites the block it mirrors.
 */
#ifndef OPENASR_GGML_HOST_H
#define OPENASR_GGML_HOST_H

#include "ggml_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

struct ggml_context;
typedef struct ggml_gallocr * ggml_gallocr_t;

/* ffi.rs:97-102 */
struct ggml_init_params {
    size_t mem_size;
    void * mem_buffer;
    bool no_alloc;
};

/* ffi.rs:57-66 */
struct ggml_tallocr {
    ggml_backend_buffer_t buffer;
    void * base;
    size_t alignment;
    size_t offset;
};

/* ---- context and tensors (ffi.rs:629-700) ---- */
struct ggml_context * ggml_init(struct ggml_init_params params);
void ggml_reset(struct ggml_context * ctx);
void ggml_free(struct ggml_context * ctx);
size_t ggml_used_mem(const struct ggml_context * ctx);
size_t ggml_get_mem_size(const struct ggml_context * ctx);
size_t ggml_tensor_overhead(void);
size_t ggml_graph_overhead_custom(size_t size, bool grads);

int64_t ggml_blck_size(enum ggml_type type);
size_t ggml_type_size(enum ggml_type type);
size_t ggml_row_size(enum ggml_type type, int64_t ne);
bool ggml_is_quantized(enum ggml_type type);
const char * ggml_type_name(enum ggml_type type);
const char * ggml_op_name(enum ggml_op op);
const char * ggml_op_desc(const struct ggml_tensor * t);

int64_t ggml_nelements(const struct ggml_tensor * t);
int64_t ggml_nrows(const struct ggml_tensor * t);
size_t ggml_nbytes(const struct ggml_tensor * t);
bool ggml_is_contiguous(const struct ggml_tensor * t);
bool ggml_is_contiguous_rows(const struct ggml_tensor * t);
bool ggml_is_transposed(const struct ggml_tensor * t);
bool ggml_is_permuted(const struct ggml_tensor * t);
bool ggml_can_repeat(const struct ggml_tensor * a, const struct ggml_tensor * b);
void * ggml_get_data(const struct ggml_tensor * t);
const char * ggml_get_name(const struct ggml_tensor * t);
struct ggml_tensor * ggml_set_name(struct ggml_tensor * t, const char * name);
struct ggml_tensor * ggml_get_first_tensor(const struct ggml_context * ctx);
struct ggml_tensor * ggml_get_next_tensor(const struct ggml_context * ctx, struct ggml_tensor * t);

struct ggml_tensor * ggml_new_tensor(struct ggml_context * ctx, enum ggml_type type, int n_dims,
                                     const int64_t * ne);
struct ggml_tensor * ggml_new_tensor_1d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0);
struct ggml_tensor * ggml_new_tensor_2d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0,
                                        int64_t ne1);
struct ggml_tensor * ggml_new_tensor_3d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0,
                                        int64_t ne1, int64_t ne2);
struct ggml_tensor * ggml_new_tensor_4d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0,
                                        int64_t ne1, int64_t ne2, int64_t ne3);
void ggml_set_input(struct ggml_tensor * t);
void ggml_set_output(struct ggml_tensor * t);

/* ---- ops on the decoder path (ffi.rs:701-1000) ---- */
struct ggml_tensor * ggml_add(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
struct ggml_tensor * ggml_sub(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
struct ggml_tensor * ggml_mul(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
struct ggml_tensor * ggml_div(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
struct ggml_tensor * ggml_scale(struct ggml_context * ctx, struct ggml_tensor * a, float s);
struct ggml_tensor * ggml_rms_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps);
struct ggml_tensor * ggml_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps);
struct ggml_tensor * ggml_silu(struct ggml_context * ctx, struct ggml_tensor * a);
struct ggml_tensor * ggml_gelu(struct ggml_context * ctx, struct ggml_tensor * a);
struct ggml_tensor * ggml_gelu_erf(struct ggml_context * ctx, struct ggml_tensor * a);
struct ggml_tensor * ggml_relu(struct ggml_context * ctx, struct ggml_tensor * a);
struct ggml_tensor * ggml_mul_mat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
void ggml_mul_mat_set_prec(struct ggml_tensor * a, enum ggml_prec prec);
struct ggml_tensor * ggml_get_rows(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
struct ggml_tensor * ggml_set_rows(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
                                   struct ggml_tensor * c);
struct ggml_tensor * ggml_argmax(struct ggml_context * ctx, struct ggml_tensor * a);
struct ggml_tensor * ggml_argmax_first(struct ggml_context * ctx, struct ggml_tensor * a);
/* ffi.rs:915-925 (ggml_conv_2d = im2col + mul_mat), cpu_graph.rs:5191-5246 */
struct ggml_tensor * ggml_im2col(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b, int s0,
                                 int s1, int p0, int p1, int d0, int d1, bool is_2D, enum ggml_type dst_type);
/* ffi.rs:915-925: kernel a [KW, KH, IC, OC] over input b [W, H, IC, N] ->
 * [OW, OH, OC, N]; IM2COL in a's type, MUL_MAT of the columns by the kernel
 * rows, then the channel-major permute and CONT */
struct ggml_tensor * ggml_conv_2d(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b, int s0,
                                  int s1, int p0, int p1, int d0, int d1);
/* ffi.rs:686-687 (the sinusoidal position tables, nn/encoder.rs:580-590) */
struct ggml_tensor * ggml_sin(struct ggml_context * ctx, struct ggml_tensor * a);
struct ggml_tensor * ggml_cos(struct ggml_context * ctx, struct ggml_tensor * a);
/* ffi.rs:724-729: a and b joined along dim */
struct ggml_tensor * ggml_concat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b, int dim);
/* ffi.rs:812: a copy of a in another type (a CPY into a new tensor) */
struct ggml_tensor * ggml_cast(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_type type);
struct ggml_tensor * ggml_soft_max(struct ggml_context * ctx, struct ggml_tensor * a);
struct ggml_tensor * ggml_soft_max_ext(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * mask,
                                       float scale, float max_bias);
struct ggml_tensor * ggml_flash_attn_ext(struct ggml_context * ctx, struct ggml_tensor * q, struct ggml_tensor * k,
                                         struct ggml_tensor * v, struct ggml_tensor * mask, float scale,
                                         float max_bias, float logit_softcap);
void ggml_flash_attn_ext_set_prec(struct ggml_tensor * a, enum ggml_prec prec);
struct ggml_tensor * ggml_rope_ext(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
                                   struct ggml_tensor * c, int n_dims, int mode, int n_ctx_orig, float freq_base,
                                   float freq_scale, float ext_factor, float attn_factor, float beta_fast,
                                   float beta_slow);
struct ggml_tensor * ggml_cpy(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
struct ggml_tensor * ggml_cont(struct ggml_context * ctx, struct ggml_tensor * a);
struct ggml_tensor * ggml_repeat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
struct ggml_tensor * ggml_repeat_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                    int64_t ne2, int64_t ne3);
struct ggml_tensor * ggml_reshape_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0);
struct ggml_tensor * ggml_reshape_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1);
struct ggml_tensor * ggml_reshape_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                     int64_t ne2);
struct ggml_tensor * ggml_reshape_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                     int64_t ne2, int64_t ne3);
struct ggml_tensor * ggml_view_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, size_t offset);
struct ggml_tensor * ggml_view_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                  size_t nb1, size_t offset);
struct ggml_tensor * ggml_view_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                  int64_t ne2, size_t nb1, size_t nb2, size_t offset);
struct ggml_tensor * ggml_view_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                  int64_t ne2, int64_t ne3, size_t nb1, size_t nb2, size_t nb3, size_t offset);
struct ggml_tensor * ggml_permute(struct ggml_context * ctx, struct ggml_tensor * a, int axis0, int axis1,
                                  int axis2, int axis3);
struct ggml_tensor * ggml_transpose(struct ggml_context * ctx, struct ggml_tensor * a);

/* ---- graphs (ffi.rs:1001-1020) ---- */
struct ggml_cgraph * ggml_new_graph(struct ggml_context * ctx);
struct ggml_cgraph * ggml_new_graph_custom(struct ggml_context * ctx, size_t size, bool grads);
void ggml_build_forward_expand(struct ggml_cgraph * cgraph, struct ggml_tensor * tensor);
int ggml_graph_n_nodes(struct ggml_cgraph * cgraph);
struct ggml_tensor * ggml_graph_node(struct ggml_cgraph * cgraph, int i);

/* ---- quantization (ffi.rs:674-682) and f16 helpers ---- */
size_t ggml_quantize_chunk(enum ggml_type type, const float * src, void * dst, int64_t start, int64_t nrows,
                           int64_t n_per_row, const float * imatrix);
float ggml_fp16_to_fp32(ggml_fp16_t h);
ggml_fp16_t ggml_fp32_to_fp16(float f);

/* ---- backend front end (ffi.rs:399-628) ---- */
ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, struct ggml_backend_buffer_i iface,
                                               void * context, size_t size);
void ggml_backend_buffer_free(ggml_backend_buffer_t buffer);
void * ggml_backend_buffer_get_base(ggml_backend_buffer_t buffer);
size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer);
size_t ggml_backend_buffer_get_alignment(ggml_backend_buffer_t buffer);
size_t ggml_backend_buffer_get_alloc_size(ggml_backend_buffer_t buffer, const struct ggml_tensor * t);
bool ggml_backend_buffer_is_host(ggml_backend_buffer_t buffer);
void ggml_backend_buffer_set_usage(ggml_backend_buffer_t buffer, enum ggml_backend_buffer_usage usage);
enum ggml_backend_buffer_usage ggml_backend_buffer_get_usage(ggml_backend_buffer_t buffer);
void ggml_backend_buffer_clear(ggml_backend_buffer_t buffer, uint8_t value);
ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t buffer);
enum ggml_status ggml_backend_buffer_init_tensor(ggml_backend_buffer_t buffer, struct ggml_tensor * t);

const char * ggml_backend_buft_name(ggml_backend_buffer_type_t buft);
ggml_backend_buffer_t ggml_backend_buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size);
size_t ggml_backend_buft_get_alignment(ggml_backend_buffer_type_t buft);
size_t ggml_backend_buft_get_max_size(ggml_backend_buffer_type_t buft);
size_t ggml_backend_buft_get_alloc_size(ggml_backend_buffer_type_t buft, const struct ggml_tensor * t);
bool ggml_backend_buft_is_host(ggml_backend_buffer_type_t buft);
ggml_backend_dev_t ggml_backend_buft_get_device(ggml_backend_buffer_type_t buft);

int ggml_backend_tensor_set(struct ggml_tensor * t, const void * data, size_t offset, size_t size);
int ggml_backend_tensor_get(const struct ggml_tensor * t, void * data, size_t offset, size_t size);
int ggml_backend_tensor_memset(struct ggml_tensor * t, uint8_t value, size_t offset, size_t size);
int ggml_backend_tensor_alloc(ggml_backend_buffer_t buffer, struct ggml_tensor * t, void * addr);
int ggml_backend_view_init(struct ggml_tensor * t);
ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors_from_buft(struct ggml_context * ctx,
                                                               ggml_backend_buffer_type_t buft);
size_t ggml_backend_alloc_ctx_tensors_from_buft_size(struct ggml_context * ctx, ggml_backend_buffer_type_t buft);
ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(struct ggml_context * ctx, ggml_backend_t backend);

const char * ggml_backend_name(ggml_backend_t backend);
void ggml_backend_free(ggml_backend_t backend);
ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend);
ggml_backend_buffer_t ggml_backend_alloc_buffer(ggml_backend_t backend, size_t size);
void ggml_backend_synchronize(ggml_backend_t backend);
enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, struct ggml_cgraph * cgraph);
enum ggml_status ggml_backend_graph_compute_async(ggml_backend_t backend, struct ggml_cgraph * cgraph);
enum ggml_status ggml_backend_graph_compute_with_abort(ggml_backend_t backend, struct ggml_cgraph * cgraph,
                                                       ggml_abort_callback abort_callback,
                                                       void * abort_callback_data,
                                                       struct ggml_backend_graph_cancel_capability * cap);
bool ggml_backend_supports_op(ggml_backend_t backend, const struct ggml_tensor * op);
ggml_backend_dev_t ggml_backend_get_device(ggml_backend_t backend);

const char * ggml_backend_dev_name(ggml_backend_dev_t dev);
const char * ggml_backend_dev_description(ggml_backend_dev_t dev);
void ggml_backend_dev_memory(ggml_backend_dev_t dev, size_t * free, size_t * total);
enum ggml_backend_dev_type ggml_backend_dev_type(ggml_backend_dev_t dev);
void ggml_backend_dev_get_props(ggml_backend_dev_t dev, struct ggml_backend_dev_props * props);
ggml_backend_reg_t ggml_backend_dev_backend_reg(ggml_backend_dev_t dev);
ggml_backend_t ggml_backend_dev_init(ggml_backend_dev_t dev, const char * params);
ggml_backend_buffer_type_t ggml_backend_dev_buffer_type(ggml_backend_dev_t dev);
ggml_backend_buffer_type_t ggml_backend_dev_host_buffer_type(ggml_backend_dev_t dev);
/* plain host memory (ggml-base's CPU buffer type) */
ggml_backend_buffer_type_t ggml_backend_cpu_buffer_type(void);
ggml_backend_buffer_t ggml_backend_dev_buffer_from_host_ptr(ggml_backend_dev_t dev, void * ptr, size_t size,
                                                            size_t max_tensor_size);
bool ggml_backend_dev_supports_op(ggml_backend_dev_t dev, const struct ggml_tensor * op);
bool ggml_backend_dev_supports_buft(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft);
bool ggml_backend_dev_offload_op(ggml_backend_dev_t dev, const struct ggml_tensor * op);

const char * ggml_backend_reg_name(ggml_backend_reg_t reg);
size_t ggml_backend_reg_dev_count(ggml_backend_reg_t reg);
ggml_backend_dev_t ggml_backend_reg_dev_get(ggml_backend_reg_t reg, size_t index);
void * ggml_backend_reg_get_proc_address(ggml_backend_reg_t reg, const char * name);

/* registry (ffi.rs:400-445, 600-612) */
void ggml_backend_register(ggml_backend_reg_t reg);
size_t ggml_backend_reg_count(void);
ggml_backend_reg_t ggml_backend_reg_get(size_t index);
size_t ggml_backend_dev_count(void);
ggml_backend_dev_t ggml_backend_dev_get(size_t index);
ggml_backend_t ggml_backend_init_by_type(enum ggml_backend_dev_type type, const char * params);
ggml_backend_t ggml_backend_init_best(void);
ggml_backend_reg_t ggml_backend_load(const char * path);
void ggml_backend_unload(ggml_backend_reg_t reg);
ggml_backend_reg_t ggml_backend_load_verified_v3_utf8(const char * path_utf8, const char * const * dependency_dirs_utf8,
                                                      size_t dependency_dir_count,
                                                      const char * expected_openasr_abi_v1,
                                                      const char * expected_provider_v1,
                                                      const char * expected_device_target,
                                                      const char * minimum_driver_version);
bool ggml_backend_probe_verified_v3_utf8(const char * path_utf8, const char * const * dependency_dirs_utf8,
                                         size_t dependency_dir_count, const char * expected_openasr_abi_v1,
                                         const char * expected_provider_v1, const char * expected_device_target,
                                         const char * minimum_driver_version, char * driver_out,
                                         size_t driver_out_capacity);
/* the host's own ABI fingerprint (the value build.rs:1145-1256 bakes into the host) */
const char * ggml_backend_host_abi_fingerprint(void);

/* ---- graph allocator (ffi.rs:565-600) ---- */
ggml_gallocr_t ggml_gallocr_new(ggml_backend_buffer_type_t buft);
void ggml_gallocr_free(ggml_gallocr_t galloc);
bool ggml_gallocr_alloc_graph(ggml_gallocr_t galloc, struct ggml_cgraph * graph);
size_t ggml_gallocr_get_buffer_size(ggml_gallocr_t galloc, int buffer_id);
struct ggml_tallocr ggml_tallocr_new(ggml_backend_buffer_t buffer);
int ggml_tallocr_alloc(struct ggml_tallocr * talloc, struct ggml_tensor * t);

#ifdef __cplusplus
}
#endif

#endif
