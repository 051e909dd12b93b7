// ggml_base.cpp -- context, tensor, op-constructor and graph part of this
// build's ggml-base (declared in include/ggml_host.h). It reproduces the
// shape inference and op_params packing of the ggml ops the OpenASR decoder
// graphs use (call sites: crates/openasr-core/src/nn/decoder.rs:1850-2145,
// models/qwen/llm_transformer.rs:2096-2115, 5169-5320,
// models/whisper/ggml_decoder_graph.rs:3869-4052), so a device plugin sees the
// same node stream the Rust host would hand it.

#include "ggml_host.h"

#include <cassert>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace {

struct obj_header {
    size_t offs;  // of the payload, from the context base
    size_t size;  // payload bytes
    obj_header * next;
    int kind;     // 0 tensor, 1 graph
};

constexpr size_t kObjSize = (sizeof(obj_header) + GGML_MEM_ALIGN - 1) / GGML_MEM_ALIGN * GGML_MEM_ALIGN;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct type_info {
    const char * name;
    int64_t blck;
    size_t size;
    bool quantized;
};

type_info type_table(enum ggml_type t) {
    switch (t) {
        case GGML_TYPE_F32: return {"f32", 1, 4, false};
        case GGML_TYPE_F16: return {"f16", 1, 2, false};
        case GGML_TYPE_BF16: return {"bf16", 1, 2, false};
        case GGML_TYPE_Q4_0: return {"q4_0", 32, 18, true};
        case GGML_TYPE_Q4_1: return {"q4_1", 32, 20, true};
        case GGML_TYPE_Q5_0: return {"q5_0", 32, 22, true};
        case GGML_TYPE_Q5_1: return {"q5_1", 32, 24, true};
        case GGML_TYPE_Q8_0: return {"q8_0", 32, 34, true};
        case GGML_TYPE_Q8_1: return {"q8_1", 32, 36, true};
        case GGML_TYPE_Q2_K: return {"q2_K", 256, 84, true};
        case GGML_TYPE_Q3_K: return {"q3_K", 256, 110, true};
        case GGML_TYPE_Q4_K: return {"q4_K", 256, 144, true};
        case GGML_TYPE_Q5_K: return {"q5_K", 256, 176, true};
        case GGML_TYPE_Q6_K: return {"q6_K", 256, 210, true};
        case GGML_TYPE_Q8_K: return {"q8_K", 256, 292, true};
        case GGML_TYPE_I8: return {"i8", 1, 1, false};
        case GGML_TYPE_I16: return {"i16", 1, 2, false};
        case GGML_TYPE_I32: return {"i32", 1, 4, false};
        case GGML_TYPE_I64: return {"i64", 1, 8, false};
        case GGML_TYPE_F64: return {"f64", 1, 8, false};
        default: return {"unknown", 0, 0, false};
    }
}

[[noreturn]] void die(const char * what) {
    std::fprintf(stderr, "ggml-base: %s\n", what);
    std::abort();
}

#define GB_REQUIRE(cond, msg) \
    do {                      \
        if (!(cond)) die(msg); \
    } while (0)

}  // namespace

struct ggml_context {
    size_t mem_size;
    char * mem;
    bool owns_mem;
    bool no_alloc;
    size_t used;
    obj_header * first;
    obj_header * last;
};

extern "C" {

// ------------------------------------------------------------------ types --

int64_t ggml_blck_size(enum ggml_type type) { return type_table(type).blck; }
size_t ggml_type_size(enum ggml_type type) { return type_table(type).size; }
bool ggml_is_quantized(enum ggml_type type) { return type_table(type).quantized; }
const char * ggml_type_name(enum ggml_type type) { return type_table(type).name; }

size_t ggml_row_size(enum ggml_type type, int64_t ne) {
    const type_info ti = type_table(type);
    GB_REQUIRE(ti.blck > 0 && ne % ti.blck == 0, "row length is not a multiple of the block size");
    return ti.size * (size_t) (ne / ti.blck);
}

static const char * const kOpNames[GGML_OP_COUNT] = {
    "NONE", "DUP", "ADD", "ADD_ID", "ADD1", "ACC", "SUB", "MUL", "DIV", "SQR", "SQRT", "LOG", "SIN", "COS", "SUM",
    "SUM_ROWS", "CUMSUM", "MEAN", "ARGMAX", "COUNT_EQUAL", "REPEAT", "REPEAT_BACK", "CONCAT", "SILU_BACK", "NORM",
    "RMS_NORM", "RMS_NORM_BACK", "GROUP_NORM", "L2_NORM", "MUL_MAT", "MUL_MAT_ID", "OUT_PROD", "SCALE", "SET",
    "CPY", "CONT", "RESHAPE", "VIEW", "PERMUTE", "TRANSPOSE", "GET_ROWS", "GET_ROWS_BACK", "SET_ROWS", "DIAG",
    "DIAG_MASK_INF", "DIAG_MASK_ZERO", "SOFT_MAX", "SOFT_MAX_BACK", "ROPE", "ROPE_BACK", "CLAMP",
    "CONV_TRANSPOSE_1D", "IM2COL", "IM2COL_BACK", "IM2COL_3D", "CONV_2D", "CONV_3D", "CONV_2D_DW",
    "CONV_TRANSPOSE_2D", "POOL_1D", "POOL_2D", "POOL_2D_BACK", "UPSCALE", "PAD", "PAD_REFLECT_1D", "ROLL",
    "ARANGE", "TIMESTEP_EMBEDDING", "ARGSORT", "LEAKY_RELU", "TRI", "FILL", "FLASH_ATTN_EXT", "FLASH_ATTN_BACK",
    "SSM_CONV", "SSM_SCAN", "WIN_PART", "WIN_UNPART", "GET_REL_POS", "ADD_REL_POS", "RWKV_WKV6",
    "GATED_LINEAR_ATTN", "RWKV_WKV7", "SOLVE_TRI", "UNARY", "MAP_CUSTOM1", "MAP_CUSTOM2", "MAP_CUSTOM3", "CUSTOM",
    "CROSS_ENTROPY_LOSS", "CROSS_ENTROPY_LOSS_BACK", "OPT_STEP_ADAMW", "OPT_STEP_SGD", "GLU", "ARGMAX_FIRST",
};

const char * ggml_op_name(enum ggml_op op) { return (op >= 0 && op < GGML_OP_COUNT) ? kOpNames[op] : "?"; }

const char * ggml_op_desc(const struct ggml_tensor * t) {
    if (t->op == GGML_OP_UNARY) {
        static const char * const unames[] = {"ABS", "SGN", "NEG", "STEP", "TANH", "ELU", "RELU", "SIGMOID",
                                              "GELU", "GELU_QUICK", "SILU", "HARDSWISH", "HARDSIGMOID", "EXP",
                                              "GELU_ERF"};
        const int u = t->op_params[0];
        return (u >= 0 && u < GGML_UNARY_OP_COUNT) ? unames[u] : "UNARY?";
    }
    return ggml_op_name(t->op);
}

// --------------------------------------------------------------- context --

struct ggml_context * ggml_init(struct ggml_init_params params) {
    ggml_context * ctx = (ggml_context *) std::calloc(1, sizeof(ggml_context));
    if (!ctx) return nullptr;
    ctx->mem_size = params.mem_size ? params.mem_size : 16 * 1024 * 1024;
    if (params.mem_buffer) {
        ctx->mem = (char *) params.mem_buffer;
        ctx->owns_mem = false;
    } else {
        ctx->mem = (char *) std::aligned_alloc(GGML_MEM_ALIGN, align_up(ctx->mem_size, GGML_MEM_ALIGN));
        ctx->owns_mem = true;
        if (!ctx->mem) {
            std::free(ctx);
            return nullptr;
        }
    }
    ctx->no_alloc = params.no_alloc;
    return ctx;
}

void ggml_reset(struct ggml_context * ctx) {
    if (!ctx) return;
    ctx->used = 0;
    ctx->first = ctx->last = nullptr;
}

void ggml_free(struct ggml_context * ctx) {
    if (!ctx) return;
    if (ctx->owns_mem) std::free(ctx->mem);
    std::free(ctx);
}

size_t ggml_used_mem(const struct ggml_context * ctx) { return ctx->used; }
size_t ggml_get_mem_size(const struct ggml_context * ctx) { return ctx->mem_size; }
size_t ggml_tensor_overhead(void) { return kObjSize + align_up(sizeof(ggml_tensor), GGML_MEM_ALIGN); }

static size_t hash_size_for(size_t n) { return 2 * n + 1; }

size_t ggml_graph_overhead_custom(size_t size, bool grads) {
    (void) grads;
    const size_t hs = hash_size_for(size);
    return kObjSize + align_up(sizeof(ggml_cgraph), GGML_MEM_ALIGN) +
           align_up(2 * size * sizeof(ggml_tensor *), GGML_MEM_ALIGN) +
           align_up(hs * sizeof(ggml_tensor *), GGML_MEM_ALIGN);
}

static void * ctx_alloc_object(ggml_context * ctx, size_t payload, int kind) {
    const size_t need = kObjSize + align_up(payload, GGML_MEM_ALIGN);
    if (ctx->used + need > ctx->mem_size) {
        std::fprintf(stderr, "ggml-base: context out of memory (need %zu, used %zu of %zu)\n", need, ctx->used,
                     ctx->mem_size);
        return nullptr;
    }
    obj_header * h = (obj_header *) (ctx->mem + ctx->used);
    h->offs = ctx->used + kObjSize;
    h->size = payload;
    h->next = nullptr;
    h->kind = kind;
    if (ctx->last) ctx->last->next = h;
    else ctx->first = h;
    ctx->last = h;
    ctx->used += need;
    return ctx->mem + h->offs;
}

// ---------------------------------------------------------------- tensors --

int64_t ggml_nelements(const struct ggml_tensor * t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
int64_t ggml_nrows(const struct ggml_tensor * t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

size_t ggml_nbytes(const struct ggml_tensor * t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] <= 0) return 0;
    }
    const int64_t blck = ggml_blck_size(t->type);
    size_t nbytes;
    if (blck == 1) {
        nbytes = ggml_type_size(t->type);
        for (int i = 0; i < GGML_MAX_DIMS; i++) nbytes += (size_t) (t->ne[i] - 1) * t->nb[i];
    } else {
        nbytes = (size_t) (t->ne[0] / blck) * t->nb[0];
        for (int i = 1; i < GGML_MAX_DIMS; i++) nbytes += (size_t) (t->ne[i] - 1) * t->nb[i];
    }
    return nbytes;
}

static bool is_contiguous_n(const ggml_tensor * t, int n) {
    size_t next = ggml_type_size(t->type);
    if (t->ne[0] != ggml_blck_size(t->type) && t->nb[0] != next) return false;
    next *= (size_t) (t->ne[0] / ggml_blck_size(t->type));
    for (int i = 1; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] != 1) {
            if (i > n) {
                if (t->nb[i] != next) return false;
                next *= (size_t) t->ne[i];
            } else {
                next = (size_t) t->ne[i] * t->nb[i];
            }
        }
    }
    return true;
}

bool ggml_is_contiguous(const struct ggml_tensor * t) { return is_contiguous_n(t, 0); }
bool ggml_is_contiguous_rows(const struct ggml_tensor * t) {
    return t->ne[0] == ggml_blck_size(t->type) || t->nb[0] == ggml_type_size(t->type);
}
bool ggml_is_transposed(const struct ggml_tensor * t) { return t->nb[0] > t->nb[1]; }
bool ggml_is_permuted(const struct ggml_tensor * t) {
    return t->nb[0] > t->nb[1] || t->nb[1] > t->nb[2] || t->nb[2] > t->nb[3];
}

bool ggml_can_repeat(const struct ggml_tensor * a, const struct ggml_tensor * b) {
    if (ggml_nelements(a) == 0) return ggml_nelements(b) == 0;
    for (int i = 0; i < GGML_MAX_DIMS; i++) {
        if (b->ne[i] % a->ne[i] != 0) return false;
    }
    return true;
}

void * ggml_get_data(const struct ggml_tensor * t) { return t->data; }
const char * ggml_get_name(const struct ggml_tensor * t) { return t->name; }

struct ggml_tensor * ggml_set_name(struct ggml_tensor * t, const char * name) {
    size_t i = 0;
    for (; i < GGML_MAX_NAME - 1 && name[i]; i++) t->name[i] = name[i];
    t->name[i] = '\0';
    return t;
}

static ggml_tensor * next_tensor_obj(obj_header * h) {
    while (h) {
        if (h->kind == 0) return (ggml_tensor *) ((char *) h + kObjSize);
        h = h->next;
    }
    return nullptr;
}

struct ggml_tensor * ggml_get_first_tensor(const struct ggml_context * ctx) { return next_tensor_obj(ctx->first); }

struct ggml_tensor * ggml_get_next_tensor(const struct ggml_context * ctx, struct ggml_tensor * t) {
    (void) ctx;
    obj_header * h = (obj_header *) ((char *) t - kObjSize);
    return next_tensor_obj(h->next);
}

static ggml_tensor * new_tensor_impl(ggml_context * ctx, enum ggml_type type, int n_dims, const int64_t * ne,
                                     ggml_tensor * view_src, size_t view_offs) {
    GB_REQUIRE(n_dims >= 1 && n_dims <= GGML_MAX_DIMS, "tensor rank out of range");
    GB_REQUIRE(type_table(type).blck > 0, "unsupported tensor type");
    if (view_src && view_src->view_src) {
        view_offs += view_src->view_offs;
        view_src = view_src->view_src;
    }
    size_t data_size = ggml_row_size(type, ne[0]);
    for (int i = 1; i < n_dims; i++) data_size *= (size_t) ne[i];
    GB_REQUIRE(view_src == nullptr || data_size == 0 || data_size + view_offs <= ggml_nbytes(view_src),
               "view exceeds its source");
    void * data = view_src ? view_src->data : nullptr;
    if (data) data = (char *) data + view_offs;
    size_t payload = sizeof(ggml_tensor);
    const bool own_data = view_src == nullptr && data == nullptr && !ctx->no_alloc;
    if (own_data) payload = align_up(sizeof(ggml_tensor), GGML_MEM_ALIGN) + data_size;
    char * p = (char *) ctx_alloc_object(ctx, payload, 0);
    if (!p) return nullptr;
    ggml_tensor * t = (ggml_tensor *) p;
    std::memset(t, 0, sizeof(*t));
    t->type = type;
    t->buffer = view_src ? view_src->buffer : nullptr;
    for (int i = 0; i < GGML_MAX_DIMS; i++) t->ne[i] = 1;
    for (int i = 0; i < n_dims; i++) t->ne[i] = ne[i];
    t->nb[0] = ggml_type_size(type);
    t->nb[1] = t->nb[0] * (size_t) (t->ne[0] / ggml_blck_size(type));
    for (int i = 2; i < GGML_MAX_DIMS; i++) t->nb[i] = t->nb[i - 1] * (size_t) t->ne[i - 1];
    t->op = GGML_OP_NONE;
    t->view_src = view_src;
    t->view_offs = view_offs;
    t->data = own_data ? p + align_up(sizeof(ggml_tensor), GGML_MEM_ALIGN) : data;
    return t;
}

struct ggml_tensor * ggml_new_tensor(struct ggml_context * ctx, enum ggml_type type, int n_dims,
                                     const int64_t * ne) {
    return new_tensor_impl(ctx, type, n_dims, ne, nullptr, 0);
}
struct ggml_tensor * ggml_new_tensor_1d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0) {
    return ggml_new_tensor(ctx, type, 1, &ne0);
}
struct ggml_tensor * ggml_new_tensor_2d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0, int64_t ne1) {
    const int64_t ne[2] = {ne0, ne1};
    return ggml_new_tensor(ctx, type, 2, ne);
}
struct ggml_tensor * ggml_new_tensor_3d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0, int64_t ne1,
                                        int64_t ne2) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    return ggml_new_tensor(ctx, type, 3, ne);
}
struct ggml_tensor * ggml_new_tensor_4d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0, int64_t ne1,
                                        int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return ggml_new_tensor(ctx, type, 4, ne);
}

void ggml_set_input(struct ggml_tensor * t) { t->flags |= GGML_TENSOR_FLAG_INPUT; }
void ggml_set_output(struct ggml_tensor * t) { t->flags |= GGML_TENSOR_FLAG_OUTPUT; }

static ggml_tensor * dup_tensor(ggml_context * ctx, const ggml_tensor * a) {
    return ggml_new_tensor(ctx, a->type, GGML_MAX_DIMS, a->ne);
}

static ggml_tensor * view_tensor(ggml_context * ctx, ggml_tensor * src) {
    ggml_tensor * r = new_tensor_impl(ctx, src->type, GGML_MAX_DIMS, src->ne, src, 0);
    if (!r) return nullptr;
    for (int i = 0; i < GGML_MAX_DIMS; i++) r->nb[i] = src->nb[i];
    return r;
}

static void set_op_params(ggml_tensor * t, const void * params, size_t size) {
    GB_REQUIRE(size <= GGML_MAX_OP_PARAMS, "op params too large");
    std::memcpy(t->op_params, params, size);
}

static void set_op_f32(ggml_tensor * t, int i, float v) { std::memcpy(&t->op_params[i], &v, sizeof(float)); }

// ------------------------------------------------------------------- ops --

static ggml_tensor * binary_op(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, enum ggml_op op) {
    GB_REQUIRE(ggml_can_repeat(b, a), "binary op: b does not broadcast into a");
    ggml_tensor * r = dup_tensor(ctx, a);
    if (!r) return nullptr;
    r->op = op;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor * ggml_add(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    return binary_op(ctx, a, b, GGML_OP_ADD);
}
struct ggml_tensor * ggml_sub(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    return binary_op(ctx, a, b, GGML_OP_SUB);
}
struct ggml_tensor * ggml_mul(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    return binary_op(ctx, a, b, GGML_OP_MUL);
}
struct ggml_tensor * ggml_div(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    return binary_op(ctx, a, b, GGML_OP_DIV);
}

struct ggml_tensor * ggml_scale(struct ggml_context * ctx, struct ggml_tensor * a, float s) {
    ggml_tensor * r = dup_tensor(ctx, a);
    if (!r) return nullptr;
    set_op_f32(r, 0, s);
    set_op_f32(r, 1, 0.0f);
    r->op = GGML_OP_SCALE;
    r->src[0] = a;
    return r;
}

static ggml_tensor * norm_op(ggml_context * ctx, ggml_tensor * a, float eps, enum ggml_op op) {
    ggml_tensor * r = dup_tensor(ctx, a);
    if (!r) return nullptr;
    set_op_f32(r, 0, eps);
    r->op = op;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_rms_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps) {
    return norm_op(ctx, a, eps, GGML_OP_RMS_NORM);
}
struct ggml_tensor * ggml_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps) {
    return norm_op(ctx, a, eps, GGML_OP_NORM);
}

static ggml_tensor * unary_op(ggml_context * ctx, ggml_tensor * a, enum ggml_unary_op u) {
    GB_REQUIRE(ggml_is_contiguous_rows(a), "unary op needs contiguous rows");
    ggml_tensor * r = dup_tensor(ctx, a);
    if (!r) return nullptr;
    r->op_params[0] = (int32_t) u;
    r->op = GGML_OP_UNARY;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_silu(struct ggml_context * ctx, struct ggml_tensor * a) {
    return unary_op(ctx, a, GGML_UNARY_OP_SILU);
}
struct ggml_tensor * ggml_gelu(struct ggml_context * ctx, struct ggml_tensor * a) {
    return unary_op(ctx, a, GGML_UNARY_OP_GELU);
}
struct ggml_tensor * ggml_gelu_erf(struct ggml_context * ctx, struct ggml_tensor * a) {
    return unary_op(ctx, a, GGML_UNARY_OP_GELU_ERF);
}
struct ggml_tensor * ggml_relu(struct ggml_context * ctx, struct ggml_tensor * a) {
    return unary_op(ctx, a, GGML_UNARY_OP_RELU);
}

struct ggml_tensor * ggml_mul_mat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    GB_REQUIRE(a->ne[0] == b->ne[0] && b->ne[2] % a->ne[2] == 0 && b->ne[3] % a->ne[3] == 0,
               "mul_mat: shapes do not contract");
    GB_REQUIRE(!ggml_is_transposed(a), "mul_mat: lhs must not be transposed");
    const int64_t ne[4] = {a->ne[1], b->ne[1], b->ne[2], b->ne[3]};
    ggml_tensor * r = ggml_new_tensor(ctx, GGML_TYPE_F32, 4, ne);
    if (!r) return nullptr;
    r->op = GGML_OP_MUL_MAT;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

void ggml_mul_mat_set_prec(struct ggml_tensor * a, enum ggml_prec prec) { a->op_params[0] = (int32_t) prec; }

struct ggml_tensor * ggml_get_rows(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    GB_REQUIRE(a->ne[2] == b->ne[1] && b->ne[3] == 1 && b->type == GGML_TYPE_I32, "get_rows: bad shapes");
    const enum ggml_type type = a->type == GGML_TYPE_I32 ? GGML_TYPE_I32 : GGML_TYPE_F32;
    ggml_tensor * r = ggml_new_tensor_4d(ctx, type, a->ne[0], b->ne[0], b->ne[1], b->ne[2]);
    if (!r) return nullptr;
    r->op = GGML_OP_GET_ROWS;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

// a: destination [n_embd, rows, ne2, ne3]; b: source [n_embd, n_rows, ne2, ne3]
// c: row indices [n_rows, ne11, ne12] broadcast over ne2/ne3
struct ggml_tensor * ggml_set_rows(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
                                   struct ggml_tensor * c) {
    GB_REQUIRE(a->ne[0] == b->ne[0] && a->ne[2] == b->ne[2] && a->ne[3] == b->ne[3], "set_rows: shape mismatch");
    GB_REQUIRE(c->ne[0] == b->ne[1] && b->ne[2] % c->ne[1] == 0 && b->ne[3] % c->ne[2] == 0 && c->ne[3] == 1,
               "set_rows: index shape mismatch");
    GB_REQUIRE(b->type == GGML_TYPE_F32 && (c->type == GGML_TYPE_I32 || c->type == GGML_TYPE_I64),
               "set_rows: types");
    ggml_tensor * r = view_tensor(ctx, a);
    if (!r) return nullptr;
    r->op = GGML_OP_SET_ROWS;
    r->src[0] = b;
    r->src[1] = c;
    return r;
}

static ggml_tensor * argmax_op(ggml_context * ctx, ggml_tensor * a, enum ggml_op op) {
    GB_REQUIRE(a->ne[2] == 1 && a->ne[3] == 1 && a->type == GGML_TYPE_F32, "argmax: needs an f32 matrix");
    ggml_tensor * r = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, a->ne[1]);
    if (!r) return nullptr;
    r->op = op;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_argmax(struct ggml_context * ctx, struct ggml_tensor * a) {
    return argmax_op(ctx, a, GGML_OP_ARGMAX);
}
struct ggml_tensor * ggml_argmax_first(struct ggml_context * ctx, struct ggml_tensor * a) {
    return argmax_op(ctx, a, GGML_OP_ARGMAX_FIRST);
}

// Output length of a strided, padded, dilated convolution along one axis.
static int64_t conv_out_len(int64_t in, int64_t k, int s, int p, int d) { return (in + 2 * p - d * (k - 1) - 1) / s + 1; }

// Column matrix of a convolution (the first half of ggml_conv_2d / conv_1d,
// used by nn/conv.rs:82-110 for the Qwen audio encoder's stem). `a` is the
// kernel [KW, KH, IC, OC] (2-D) or [K, IC, OC] (1-D), read for its shape only;
// `b` the input [IW, IH, IC, N] or [IW, IC, N]. The result row for output
// pixel (n, oh, ow) holds IC*KH*KW taps, ic-major then kh then kw, zero where
// the tap falls into padding. op_params = {s0, s1, p0, p1, d0, d1, is_2D}.
struct ggml_tensor * ggml_im2col(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b, int s0,
                                 int s1, int p0, int p1, int d0, int d1, bool is_2D, enum ggml_type dst_type) {
    GB_REQUIRE(s0 > 0 && d0 > 0 && p0 >= 0 && (!is_2D || (s1 > 0 && d1 > 0 && p1 >= 0)),
               "im2col: bad stride/padding/dilation");
    GB_REQUIRE(dst_type == GGML_TYPE_F16 || dst_type == GGML_TYPE_F32, "im2col: result must be f16 or f32");
    int64_t ne[4];
    if (is_2D) {
        GB_REQUIRE(a->ne[2] == b->ne[2], "im2col: kernel and input channel counts differ");
        const int64_t oh = conv_out_len(b->ne[1], a->ne[1], s1, p1, d1);
        const int64_t ow = conv_out_len(b->ne[0], a->ne[0], s0, p0, d0);
        GB_REQUIRE(oh > 0 && ow > 0, "im2col: kernel larger than padded input");
        ne[0] = a->ne[2] * a->ne[1] * a->ne[0], ne[1] = ow, ne[2] = oh, ne[3] = b->ne[3];
    } else {
        GB_REQUIRE(a->ne[1] == b->ne[1] && b->ne[3] == 1, "im2col: kernel and input channel counts differ");
        const int64_t ow = conv_out_len(b->ne[0], a->ne[0], s0, p0, d0);
        GB_REQUIRE(ow > 0, "im2col: kernel larger than padded input");
        ne[0] = a->ne[1] * a->ne[0], ne[1] = ow, ne[2] = b->ne[2], ne[3] = 1;
    }
    ggml_tensor * r = new_tensor_impl(ctx, dst_type, 4, ne, nullptr, 0);
    if (!r) return nullptr;
    const int32_t params[7] = {s0, s1, p0, p1, d0, d1, is_2D ? 1 : 0};
    set_op_params(r, params, sizeof(params));
    r->op = GGML_OP_IM2COL;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor * ggml_conv_2d(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b, int s0,
                                  int s1, int p0, int p1, int d0, int d1) {
    // columns [IC KH KW, OW, OH, N] in the kernel's type; the columns are the
    // MUL_MAT's first operand and the kernel rows its second, so the product
    // is [OW OH N, OC]
    ggml_tensor * im = ggml_im2col(ctx, a, b, s0, s1, p0, p1, d0, d1, true, a->type);
    if (!im) return nullptr;
    ggml_tensor * r = ggml_mul_mat(ctx, ggml_reshape_2d(ctx, im, im->ne[0], im->ne[3] * im->ne[2] * im->ne[1]),
                                   ggml_reshape_2d(ctx, a, a->ne[0] * a->ne[1] * a->ne[2], a->ne[3]));
    if (!r) return nullptr;
    r = ggml_reshape_4d(ctx, r, im->ne[1], im->ne[2], im->ne[3], a->ne[3]);  // [OW, OH, N, OC]
    return ggml_cont(ctx, ggml_permute(ctx, r, 0, 1, 3, 2));                  // [OW, OH, OC, N]
}

struct ggml_tensor * ggml_soft_max_ext(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * mask,
                                       float scale, float max_bias) {
    GB_REQUIRE(ggml_is_contiguous(a), "soft_max: input must be contiguous");
    if (mask) {
        GB_REQUIRE(mask->ne[0] == a->ne[0] && mask->ne[1] >= a->ne[1] && a->ne[2] % mask->ne[2] == 0 &&
                       a->ne[3] % mask->ne[3] == 0,
                   "soft_max: mask shape");
    }
    ggml_tensor * r = dup_tensor(ctx, a);
    if (!r) return nullptr;
    set_op_f32(r, 0, scale);
    set_op_f32(r, 1, max_bias);
    r->op = GGML_OP_SOFT_MAX;
    r->src[0] = a;
    r->src[1] = mask;
    return r;
}

struct ggml_tensor * ggml_soft_max(struct ggml_context * ctx, struct ggml_tensor * a) {
    return ggml_soft_max_ext(ctx, a, nullptr, 1.0f, 0.0f);
}

// q [D, n_q, Hq, n_seq]; k,v [D, n_kv, Hkv, n_seq]; mask [n_kv, >=n_q, 1|.., 1|n_seq]
// result [Dv, Hq, n_q, n_seq]
struct ggml_tensor * ggml_flash_attn_ext(struct ggml_context * ctx, struct ggml_tensor * q, struct ggml_tensor * k,
                                         struct ggml_tensor * v, struct ggml_tensor * mask, float scale,
                                         float max_bias, float logit_softcap) {
    GB_REQUIRE(q->ne[0] == k->ne[0] && k->ne[1] == v->ne[1], "flash_attn_ext: q/k/v shapes");
    GB_REQUIRE(q->ne[2] % k->ne[2] == 0 && q->ne[3] % k->ne[3] == 0, "flash_attn_ext: head broadcast");
    if (mask) {
        GB_REQUIRE(mask->ne[0] == k->ne[1] && mask->ne[1] >= q->ne[1] && q->ne[2] % mask->ne[2] == 0 &&
                       q->ne[3] % mask->ne[3] == 0,
                   "flash_attn_ext: mask shape");
    }
    const int64_t ne[4] = {v->ne[0], q->ne[2], q->ne[1], q->ne[3]};
    ggml_tensor * r = ggml_new_tensor(ctx, GGML_TYPE_F32, 4, ne);
    if (!r) return nullptr;
    set_op_f32(r, 0, scale);
    set_op_f32(r, 1, max_bias);
    set_op_f32(r, 2, logit_softcap);
    r->op = GGML_OP_FLASH_ATTN_EXT;
    r->src[0] = q;
    r->src[1] = k;
    r->src[2] = v;
    r->src[3] = mask;
    return r;
}

void ggml_flash_attn_ext_set_prec(struct ggml_tensor * a, enum ggml_prec prec) { a->op_params[3] = (int32_t) prec; }

// op_params: {n_past=0, n_dims, mode, n_ctx=0, n_ctx_orig, freq_base, freq_scale,
//             ext_factor, attn_factor, beta_fast, beta_slow}
struct ggml_tensor * ggml_rope_ext(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
                                   struct ggml_tensor * c, int n_dims, int mode, int n_ctx_orig, float freq_base,
                                   float freq_scale, float ext_factor, float attn_factor, float beta_fast,
                                   float beta_slow) {
    GB_REQUIRE(b->type == GGML_TYPE_I32 && b->ne[0] == a->ne[2], "rope: positions must be i32 [ne2]");
    ggml_tensor * r = dup_tensor(ctx, a);
    if (!r) return nullptr;
    int32_t params[15] = {0, n_dims, mode, 0, n_ctx_orig};
    std::memcpy(params + 5, &freq_base, 4);
    std::memcpy(params + 6, &freq_scale, 4);
    std::memcpy(params + 7, &ext_factor, 4);
    std::memcpy(params + 8, &attn_factor, 4);
    std::memcpy(params + 9, &beta_fast, 4);
    std::memcpy(params + 10, &beta_slow, 4);
    set_op_params(r, params, sizeof(params));
    r->op = GGML_OP_ROPE;
    r->src[0] = a;
    r->src[1] = b;
    r->src[2] = c;
    return r;
}

struct ggml_tensor * ggml_cpy(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    GB_REQUIRE(ggml_nelements(a) == ggml_nelements(b), "cpy: element counts differ");
    ggml_tensor * r = view_tensor(ctx, b);
    if (!r) return nullptr;
    r->op = GGML_OP_CPY;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor * ggml_cast(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_type type) {
    ggml_tensor * r = ggml_new_tensor(ctx, type, GGML_MAX_DIMS, a->ne);
    if (!r) return nullptr;
    r->op = GGML_OP_CPY;
    r->src[0] = a;
    r->src[1] = r;
    return r;
}

static ggml_tensor * elementwise_op(ggml_context * ctx, ggml_tensor * a, enum ggml_op op) {
    ggml_tensor * r = dup_tensor(ctx, a);
    if (!r) return nullptr;
    r->op = op;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_sin(struct ggml_context * ctx, struct ggml_tensor * a) {
    return elementwise_op(ctx, a, GGML_OP_SIN);
}
struct ggml_tensor * ggml_cos(struct ggml_context * ctx, struct ggml_tensor * a) {
    return elementwise_op(ctx, a, GGML_OP_COS);
}

struct ggml_tensor * ggml_concat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b, int dim) {
    GB_REQUIRE(dim >= 0 && dim < GGML_MAX_DIMS && a->type == b->type, "concat: dim out of range or types differ");
    int64_t ne[GGML_MAX_DIMS];
    for (int d = 0; d < GGML_MAX_DIMS; d++) {
        GB_REQUIRE(d == dim || a->ne[d] == b->ne[d], "concat: shapes differ off the joined dim");
        ne[d] = d == dim ? a->ne[d] + b->ne[d] : a->ne[d];
    }
    ggml_tensor * r = ggml_new_tensor(ctx, a->type, GGML_MAX_DIMS, ne);
    if (!r) return nullptr;
    r->op_params[0] = dim;
    r->op = GGML_OP_CONCAT;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

// REPEAT: b's shape filled with copies of a (every dim of b a multiple of
// a's), dst[i] = a[i mod a.ne] per dim
struct ggml_tensor * ggml_repeat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    GB_REQUIRE(ggml_can_repeat(a, b), "repeat: b's shape is not a multiple of a's");
    ggml_tensor * r = ggml_new_tensor(ctx, a->type, GGML_MAX_DIMS, b->ne);
    if (!r) return nullptr;
    r->op = GGML_OP_REPEAT;
    r->src[0] = a;
    return r;
}

// REPEAT to an explicit shape (the GQA K/V expansion, nn/decoder.rs:1799-1841)
struct ggml_tensor * ggml_repeat_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                    int64_t ne2, int64_t ne3) {
    const bool empty = ggml_nelements(a) == 0;
    GB_REQUIRE(empty || (a->ne[0] > 0 && a->ne[1] > 0 && a->ne[2] > 0 && a->ne[3] > 0 && ne0 % a->ne[0] == 0 &&
                         ne1 % a->ne[1] == 0 && ne2 % a->ne[2] == 0 && ne3 % a->ne[3] == 0),
               "repeat_4d: the shape is not a multiple of the source's");
    ggml_tensor * r = ggml_new_tensor_4d(ctx, a->type, ne0, ne1, ne2, ne3);
    if (!r) return nullptr;
    r->op = GGML_OP_REPEAT;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_cont(struct ggml_context * ctx, struct ggml_tensor * a) {
    ggml_tensor * r = dup_tensor(ctx, a);
    if (!r) return nullptr;
    r->op = GGML_OP_CONT;
    r->src[0] = a;
    return r;
}

static ggml_tensor * reshape_impl(ggml_context * ctx, ggml_tensor * a, int n_dims, const int64_t * ne) {
    GB_REQUIRE(ggml_is_contiguous(a), "reshape: source must be contiguous");
    int64_t n = 1;
    for (int i = 0; i < n_dims; i++) n *= ne[i];
    GB_REQUIRE(n == ggml_nelements(a), "reshape: element count changes");
    ggml_tensor * r = new_tensor_impl(ctx, a->type, n_dims, ne, a, 0);
    if (!r) return nullptr;
    r->op = GGML_OP_RESHAPE;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_reshape_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0) {
    return reshape_impl(ctx, a, 1, &ne0);
}
struct ggml_tensor * ggml_reshape_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1) {
    const int64_t ne[2] = {ne0, ne1};
    return reshape_impl(ctx, a, 2, ne);
}
struct ggml_tensor * ggml_reshape_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                     int64_t ne2) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    return reshape_impl(ctx, a, 3, ne);
}
struct ggml_tensor * ggml_reshape_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                     int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return reshape_impl(ctx, a, 4, ne);
}

static ggml_tensor * view_impl(ggml_context * ctx, ggml_tensor * a, int n_dims, const int64_t * ne, size_t offset) {
    ggml_tensor * r = new_tensor_impl(ctx, a->type, n_dims, ne, a, offset);
    if (!r) return nullptr;
    set_op_params(r, &offset, sizeof(offset));
    r->op = GGML_OP_VIEW;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_view_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, size_t offset) {
    return view_impl(ctx, a, 1, &ne0, offset);
}
struct ggml_tensor * ggml_view_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                  size_t nb1, size_t offset) {
    const int64_t ne[2] = {ne0, ne1};
    ggml_tensor * r = view_impl(ctx, a, 2, ne, offset);
    if (!r) return nullptr;
    r->nb[1] = nb1;
    r->nb[2] = r->nb[1] * (size_t) ne1;
    r->nb[3] = r->nb[2];
    return r;
}
struct ggml_tensor * ggml_view_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                  int64_t ne2, size_t nb1, size_t nb2, size_t offset) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    ggml_tensor * r = view_impl(ctx, a, 3, ne, offset);
    if (!r) return nullptr;
    r->nb[1] = nb1;
    r->nb[2] = nb2;
    r->nb[3] = r->nb[2] * (size_t) ne2;
    return r;
}
struct ggml_tensor * ggml_view_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1,
                                  int64_t ne2, int64_t ne3, size_t nb1, size_t nb2, size_t nb3, size_t offset) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    ggml_tensor * r = view_impl(ctx, a, 4, ne, offset);
    if (!r) return nullptr;
    r->nb[1] = nb1;
    r->nb[2] = nb2;
    r->nb[3] = nb3;
    return r;
}

// ggml_permute: source dim i moves to position axis_i
struct ggml_tensor * ggml_permute(struct ggml_context * ctx, struct ggml_tensor * a, int axis0, int axis1,
                                  int axis2, int axis3) {
    const int ax[4] = {axis0, axis1, axis2, axis3};
    for (int i = 0; i < 4; i++) GB_REQUIRE(ax[i] >= 0 && ax[i] < 4, "permute: axis out of range");
    GB_REQUIRE(axis0 != axis1 && axis0 != axis2 && axis0 != axis3 && axis1 != axis2 && axis1 != axis3 &&
                   axis2 != axis3,
               "permute: axes must be distinct");
    ggml_tensor * r = view_tensor(ctx, a);
    if (!r) return nullptr;
    int64_t ne[4];
    size_t nb[4];
    for (int i = 0; i < 4; i++) {
        ne[ax[i]] = a->ne[i];
        nb[ax[i]] = a->nb[i];
    }
    for (int i = 0; i < 4; i++) {
        r->ne[i] = ne[i];
        r->nb[i] = nb[i];
    }
    r->op = GGML_OP_PERMUTE;
    r->src[0] = a;
    set_op_params(r, ax, sizeof(ax));
    return r;
}

struct ggml_tensor * ggml_transpose(struct ggml_context * ctx, struct ggml_tensor * a) {
    ggml_tensor * r = view_tensor(ctx, a);
    if (!r) return nullptr;
    r->ne[0] = a->ne[1];
    r->ne[1] = a->ne[0];
    r->nb[0] = a->nb[1];
    r->nb[1] = a->nb[0];
    r->op = GGML_OP_TRANSPOSE;
    r->src[0] = a;
    return r;
}

// ---------------------------------------------------------------- graphs --

static size_t ptr_hash(const void * p, size_t n) { return ((uintptr_t) p >> 4) % n; }

// returns true if inserted, false if already present
static bool hash_insert(ggml_hash_set * hs, ggml_tensor * t) {
    size_t i = ptr_hash(t, hs->size);
    for (size_t probes = 0; probes < hs->size; probes++) {
        if (hs->keys[i] == t) return false;
        if (hs->keys[i] == nullptr) {
            hs->keys[i] = t;
            return true;
        }
        i = (i + 1) % hs->size;
    }
    die("graph hash set full");
}

struct ggml_cgraph * ggml_new_graph_custom(struct ggml_context * ctx, size_t size, bool grads) {
    (void) grads;
    const size_t hs = hash_size_for(size);
    const size_t payload = align_up(sizeof(ggml_cgraph), GGML_MEM_ALIGN) +
                           align_up(2 * size * sizeof(ggml_tensor *), GGML_MEM_ALIGN) +
                           align_up(hs * sizeof(ggml_tensor *), GGML_MEM_ALIGN);
    char * p = (char *) ctx_alloc_object(ctx, payload, 1);
    if (!p) return nullptr;
    std::memset(p, 0, payload);
    ggml_cgraph * g = (ggml_cgraph *) p;
    char * arrays = p + align_up(sizeof(ggml_cgraph), GGML_MEM_ALIGN);
    g->size = (int) size;
    g->nodes = (ggml_tensor **) arrays;
    g->leafs = g->nodes + size;
    g->visited_hash_set.size = hs;
    g->visited_hash_set.keys = (ggml_tensor **) (arrays + align_up(2 * size * sizeof(ggml_tensor *), GGML_MEM_ALIGN));
    g->order = GGML_CGRAPH_EVAL_ORDER_LEFT_TO_RIGHT;
    return g;
}

struct ggml_cgraph * ggml_new_graph(struct ggml_context * ctx) { return ggml_new_graph_custom(ctx, 2048, false); }

static void visit_parents(ggml_cgraph * g, ggml_tensor * t) {
    if (!hash_insert(&g->visited_hash_set, t)) return;
    for (int i = 0; i < GGML_MAX_SRC; i++) {
        if (t->src[i]) visit_parents(g, t->src[i]);
    }
    if (t->op == GGML_OP_NONE && !(t->flags & GGML_TENSOR_FLAG_PARAM)) {
        GB_REQUIRE(g->n_leafs < g->size, "graph leaf capacity exceeded");
        g->leafs[g->n_leafs++] = t;
    } else {
        GB_REQUIRE(g->n_nodes < g->size, "graph node capacity exceeded");
        g->nodes[g->n_nodes++] = t;
    }
}

void ggml_build_forward_expand(struct ggml_cgraph * cgraph, struct ggml_tensor * tensor) {
    visit_parents(cgraph, tensor);
}

int ggml_graph_n_nodes(struct ggml_cgraph * cgraph) { return cgraph->n_nodes; }

struct ggml_tensor * ggml_graph_node(struct ggml_cgraph * cgraph, int i) {
    if (i < 0) i += cgraph->n_nodes;
    GB_REQUIRE(i >= 0 && i < cgraph->n_nodes, "graph node index out of range");
    return cgraph->nodes[i];
}

}  // extern "C"
