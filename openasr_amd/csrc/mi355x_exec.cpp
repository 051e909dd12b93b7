// mi355x_exec.cpp -- graph executor of the gfx950 backend.
//
// ggml hands the backend one graph per compute call
// (crates/openasr-core/src/ggml_runtime/cpu_graph.rs:8007-8055 ->
// ggml_backend_graph_compute_with_abort, ffi.rs:453-459). The executor
//   1. plans the node stream into launches: view ops are free, RMSNorm/
//      LayerNorm absorb their weight multiply and bias add, SiLU absorbs the
//      gate multiply, consecutive MUL_MATs that read the same activations
//      quantize them once;
//   2. runs the plan eagerly the first time a graph is seen and captures it
//      into a HIP graph the second time, replaying the captured graph for
//      every later identical compute (the decoder step graph is persistent
//      and only its input tensors change, llm_transformer.rs:5169-5320).
// Scratch memory (quantized activations, attention partials) is one device
// arena owned by the backend and addressed by offset, so a reallocation
// only invalidates captured graphs, never the plan.

#include "mi355x_exec.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <unordered_map>
#include <unordered_set>

#include "ggml_host.h"
#include "ops.h"

namespace mi355x {

namespace {

constexpr size_t kAlign = 256;
size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// scratch arena: [activation region][general region]
// (a compute given caller scratch points the plan at that instead of the arena)
char * arena(const backend_state * be) { return be->scratch_override ? be->scratch_override : be->scratch; }
size_t gen_offset(const backend_state * be) { return be->scratch_override ? be->override_gen_off : be->gen_off; }
char * act_base(const backend_state * be) { return arena(be); }
// the general region starts with the decode step's rope table (kept for the
// whole graph); the rest is per-launch scratch
constexpr size_t kRopeTableBytes = 64 * 1024;
char * rope_base(const backend_state * be) { return arena(be) + gen_offset(be); }
char * gen_base(const backend_state * be) { return arena(be) + gen_offset(be) + kRopeTableBytes; }

bool is_view_op(enum ggml_op op) {
    return op == GGML_OP_NONE || op == GGML_OP_RESHAPE || op == GGML_OP_VIEW || op == GGML_OP_PERMUTE ||
           op == GGML_OP_TRANSPOSE;
}

float op_f32(const ggml_tensor * t, int i) {
    float v;
    std::memcpy(&v, &t->op_params[i], sizeof(float));
    return v;
}

int64_t nelem(const ggml_tensor * t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }

bool rows_contiguous(const ggml_tensor * t, size_t esize) { return (size_t) t->nb[0] == esize; }

bool is_contiguous(const ggml_tensor * t) {
    size_t expect = 0;
    int64_t blck = 1;
    switch (t->type) {
        case GGML_TYPE_F32: expect = 4; break;
        case GGML_TYPE_F16: expect = 2; break;
        case GGML_TYPE_I32: expect = 4; break;
        case GGML_TYPE_Q8_0: expect = 34; blck = 32; break;
        case GGML_TYPE_Q4_K: expect = 144; blck = 256; break;
        case GGML_TYPE_Q3_K: expect = 110; blck = 256; break;
        default: return false;
    }
    if (t->ne[0] % blck) return false;
    size_t next = expect * (size_t) (t->ne[0] / blck);
    if (t->ne[0] != blck && (size_t) t->nb[0] != expect) return false;
    for (int i = 1; i < 4; i++) {
        if (t->ne[i] != 1 && (size_t) t->nb[i] != next) return false;
        next *= (size_t) t->ne[i];
    }
    return true;
}

// columns of a [K, ne1, ne2, ne3] f32 activation must be uniformly strided
bool columns_foldable(const ggml_tensor * t) {
    if (t->nb[0] != 4) return false;
    if (t->ne[2] > 1 && t->nb[2] != t->nb[1] * t->ne[1]) return false;
    if (t->ne[3] > 1 && t->nb[3] != t->nb[2] * t->ne[2]) return false;
    return true;
}

// x is a view (or the tensor itself) of c, a contiguous f32 CONT of the 2-D
// view s whose rows are contiguous. Express x as a strided view of s: dims
// whose stride is a whole number of s rows move across rows, the others must
// stay inside one row from x's starting column.
bool remap_through_cont(const ggml_tensor * x, const ggml_tensor * c, const ggml_tensor * s, tview & out) {
    const int64_t off = (int64_t) ((const char *) x->data - (const char *) c->data);
    if (off < 0 || off % 4 != 0) return false;
    const int64_t row = s->ne[0];
    const int64_t base = off / 4;
    int64_t reach = base % row;  // furthest column touched by in-row dims
    out.data = (char *) s->data + (base % row) * 4 + (base / row) * (int64_t) s->nb[1];
    for (int d = 0; d < 4; d++) {
        out.ne[d] = x->ne[d];
        if (x->nb[d] % 4 != 0) return false;
        const int64_t se = (int64_t) x->nb[d] / 4;
        if (x->ne[d] == 1) {
            out.nb[d] = (int64_t) x->nb[d];
        } else if (se % row == 0) {
            out.nb[d] = (se / row) * (int64_t) s->nb[1];
        } else {
            out.nb[d] = se * 4;
            reach += se * (x->ne[d] - 1);
        }
    }
    return reach < row;
}

uint64_t mix(uint64_t h, uint64_t v) {
    h ^= v + 0x9e3779b97f4a7c15ULL + (h << 6) + (h >> 2);
    return h;
}

uint64_t tensor_sig(uint64_t h, const ggml_tensor * t) {
    h = mix(h, (uint64_t) (uintptr_t) t->data);
    h = mix(h, (uint64_t) t->type | ((uint64_t) t->op << 32));
    for (int i = 0; i < 4; i++) {
        h = mix(h, (uint64_t) t->ne[i]);
        h = mix(h, (uint64_t) t->nb[i]);
    }
    return h;
}

uint64_t graph_key(const ggml_cgraph * cg) {
    uint64_t h = mix(0x12345678ULL, (uint64_t) cg->n_nodes);
    for (int i = 0; i < cg->n_nodes; i++) {
        const ggml_tensor * t = cg->nodes[i];
        h = tensor_sig(h, t);
        for (int p = 0; p < 16; p++) h = mix(h, (uint64_t) (uint32_t) t->op_params[p]);
        for (int s = 0; s < GGML_MAX_SRC; s++) {
            if (t->src[s]) h = tensor_sig(h, t->src[s]);
        }
    }
    return h;
}

// byte range [lo, hi) of a tensor's data (its view extent)
struct span {
    uintptr_t lo = 0, hi = 0;
};

span span_of(const ggml_tensor * x) {
    span s;
    if (!x || !x->data) return s;
    s.lo = (uintptr_t) x->data;
    s.hi = s.lo + ggml_nbytes(x);
    return s;
}

span span_of(const tview & v, int64_t elem) {
    span s;
    s.lo = (uintptr_t) v.data;
    int64_t last = elem;
    for (int d = 0; d < 4; d++) last += (v.ne[d] - 1) * v.nb[d];
    s.hi = s.lo + (uintptr_t) last;
    return s;
}

bool overlap(span a, span b) { return a.lo < a.hi && b.lo < b.hi && a.lo < b.hi && b.lo < a.hi; }

// The GQA expansion of expand_attention_kv (nn/decoder.rs:1799-1841): x is
// the [D, T, g * H, 1] reshape of R = REPEAT [D, T, g, H] of S [D, T, 1, H],
// so head h of x is head h / g of S -- the broadcast FLASH_ATTN_EXT and
// MUL_MAT make natively. Gives R and S seen as [D, T, H, 1].
bool match_gqa(const ggml_tensor * x, const ggml_tensor *& rep, tview & folded) {
    const ggml_tensor * r = x->view_src ? x->view_src : x;
    if (r->op != GGML_OP_REPEAT || x == r || x->op != GGML_OP_RESHAPE || x->data != r->data) return false;
    const ggml_tensor * s = r->src[0];
    if (!s || s->type != r->type || !is_contiguous(x) || !is_contiguous(r)) return false;
    if (x->ne[0] != r->ne[0] || x->ne[1] != r->ne[1] || x->ne[2] != r->ne[2] * r->ne[3] || x->ne[3] != 1) return false;
    if (s->ne[0] != r->ne[0] || s->ne[1] != r->ne[1] || s->ne[2] != 1 || s->ne[3] != r->ne[3]) return false;
    rep = r;
    folded = make_view(s);
    folded.ne[2] = s->ne[3];
    folded.ne[3] = 1;
    folded.nb[2] = s->nb[3];
    folded.nb[3] = s->nb[3] * s->ne[3];
    return true;
}

// A launch at graph position i that also does the work of later nodes (a
// folded residual ADD, the SwiGLU pair, sibling projections) writes their
// results before the nodes in between run, and reads their inputs early.
struct hoist {
    std::vector<const ggml_tensor *> nodes;  // later nodes whose work the launch does
    std::vector<span> reads;                 // everything the launch reads
    std::vector<span> writes;                // everything it writes
    // (written, read) tensor pairs one lane reads then writes element by
    // element: they may coincide exactly (an in-place residual), not overlap
    std::vector<std::pair<const ggml_tensor *, const ggml_tensor *>> inplace;
};

// fusions a previous planning pass found unsafe under the graph's
// allocation, or that a reader could not take (see validate and replan)
struct plan_exclusions {
    std::unordered_set<const ggml_tensor *> no_bypass, no_defer, no_divert, no_fold, no_naive;
};

struct planner {
    backend_state * be;
    const ggml_cgraph * cg;
    std::unordered_map<const ggml_tensor *, int> uses;
    std::unordered_map<const ggml_tensor *, const ggml_tensor *> deferred;  // producer -> consumer it fuses into
    std::vector<step> steps;
    size_t act_need = 0;
    size_t gen_need = 0;
    const ggml_tensor * act_src = nullptr;  // activations currently quantized in the act region
    int act_wtype = -1;
    std::string error;
    int n_cu;

    // CONTs that must be materialised, unary nodes that must run at their
    // own position (validate)
    std::unordered_set<const ggml_tensor *> no_bypass, no_defer;
    // nodes whose result is consumed only in a form a fused launch wrote to
    // scratch (the attention output quantized for the output projection):
    // their own bytes are never written, so nothing else may read them
    std::unordered_set<const ggml_tensor *> unwritten;
    // attention outputs that must be written after all: a reader found one
    // unwritten, and the graph is planned again without that diversion
    std::unordered_set<const ggml_tensor *> no_divert;
    // REPEATs to materialise, unfused attention chains to run op by op
    std::unordered_set<const ggml_tensor *> no_fold, no_naive;
    bool replan = false;
    plan_exclusions exclusions() const { return {no_bypass, no_defer, no_divert, no_fold, no_naive}; }

    // GQA expansions (match_gqa) every reader of which reads the source's kv
    // heads instead: the REPEAT is not launched
    std::unordered_set<const ggml_tensor *> gqa_skip;
    // x read through a skipped REPEAT: the view of its source
    bool gqa_fold(const ggml_tensor * x, tview & v) const {
        const ggml_tensor * r = nullptr;
        return match_gqa(x, r, v) && gqa_skip.count(r);
    }
    // The unfused attention chain (nn/decoder.rs:2154-2200) as one launch at
    // its output CONT: the scores MUL_MAT S, the SOFT_MAX P, the V^T CONT VT
    // and the context MUL_MAT C are not launched on their own.
    struct naive_job {
        const ggml_tensor *S = nullptr, *P = nullptr, *VT = nullptr, *C = nullptr, *O = nullptr;
        naive_attn_args a{};
        std::vector<std::pair<span, int>> reads;  // what the launch reads, and where the graph read it
    };
    std::unordered_map<const ggml_tensor *, naive_job> naive_jobs;  // by output CONT
    std::unordered_set<const ggml_tensor *> naive_nodes;            // S, P, VT, C of the jobs
    // IM2COL results written in the bf16 hi / lo layout for their column
    // GEMM (im2col_args::split), which reads them as such
    std::unordered_set<const ggml_tensor *> split_cols;
    void find_naive();
    void find_gqa_skip();
    bool plan_naive(int i, const ggml_tensor * t);
    struct fold_read {
        const ggml_tensor * rep;
        span src;       // the expansion's source
        int from, to;   // the REPEAT's position, its last reader's
    };
    std::vector<fold_read> fold_reads;
    bool naive_dropped = false;
    bool reads_unwritten(const ggml_tensor * t, const ggml_tensor * x) {
        const ggml_tensor * r = root_of(x);
        if (!unwritten.count(r)) return false;
        no_divert.insert(r);
        replan = true;
        fail(t, "reads an output a fused launch never wrote");
        return true;
    }
    int cur = -1;  // graph position being planned

    planner(backend_state * b, const ggml_cgraph * g, const plan_exclusions & x = {})
        : be(b), cg(g), n_cu(b->dev->n_cu), no_bypass(x.no_bypass), no_defer(x.no_defer), no_divert(x.no_divert),
          no_fold(x.no_fold), no_naive(x.no_naive) {}

    std::unordered_map<const ggml_tensor *, int> index;  // node -> position in the graph
    // CONT nodes whose copy is skipped: consumers read the CONT's strided
    // source directly (CONT -> its source)
    std::unordered_map<const ggml_tensor *, const ggml_tensor *> bypass;
    std::unordered_map<const ggml_tensor *, int> bypass_last;  // bypassed CONT -> position of its last reader
    // unary nodes evaluated inside a later consumer: (node, consumer position)
    std::vector<std::pair<const ggml_tensor *, int>> deferred_unary;

    static const ggml_tensor * root_of(const ggml_tensor * x) { return x->view_src ? x->view_src : x; }

    // the view a kernel reads for tensor x (through a bypassed CONT if any)
    tview view_of(const ggml_tensor * x) const {
        auto it = bypass.find(root_of(x));
        tview v = make_view(x);
        if (it != bypass.end()) remap_through_cont(x, it->first, it->second, v);
        return v;
    }

    // A CONT of a 2-D row-contiguous f32 view is not materialised when every
    // reader is an op whose kernel takes arbitrary strides and each read view
    // maps onto the source (the column views of the fused QKV projection,
    // nn/decoder.rs:1722-1789, are made contiguous only to be reshaped).
    void find_bypass() {
        for (int i = 0; i < cg->n_nodes; i++) {
            const ggml_tensor * c = cg->nodes[i];
            if (c->op != GGML_OP_CONT || c->type != GGML_TYPE_F32 || (c->flags & GGML_TENSOR_FLAG_OUTPUT)) continue;
            if (no_bypass.count(c)) continue;
            const ggml_tensor * s = c->src[0];
            if (s->type != GGML_TYPE_F32 || s->nb[0] != 4 || s->ne[2] != 1 || s->ne[3] != 1) continue;
            if (s->nb[1] % 4 != 0) continue;
            bool ok = true, any = false;
            int last = i;
            for (int j = i + 1; j < cg->n_nodes && ok; j++) {
                const ggml_tensor * n = cg->nodes[j];
                for (int k = 0; k < GGML_MAX_SRC && ok; k++) {
                    const ggml_tensor * x = n->src[k];
                    if (!x || root_of(x) != c) continue;
                    if (is_view_op(n->op)) continue;  // metadata; its readers are checked themselves
                    any = true;
                    last = j;
                    const bool reader = n->op == GGML_OP_RMS_NORM || n->op == GGML_OP_NORM || n->op == GGML_OP_ROPE ||
                                        (n->op == GGML_OP_SET_ROWS && k == 0) ||
                                        ((n->op == GGML_OP_CPY || n->op == GGML_OP_CONT) && k == 0) ||
                                        n->op == GGML_OP_ADD || n->op == GGML_OP_MUL || n->op == GGML_OP_SUB ||
                                        n->op == GGML_OP_DIV;
                    tview v;
                    ok = reader && remap_through_cont(x, c, s, v);
                }
            }
            if (ok && any) {
                bypass[c] = s;
                bypass_last[c] = last;
            }
        }
    }

    void count_uses() {
        for (int i = 0; i < cg->n_nodes; i++) {
            index[cg->nodes[i]] = i;
            for (int s = 0; s < GGML_MAX_SRC; s++) {
                if (cg->nodes[i]->src[s]) uses[cg->nodes[i]->src[s]]++;
            }
        }
    }

    bool single_use(const ggml_tensor * t) const {
        auto it = uses.find(t);
        return it != uses.end() && it->second == 1 && !(t->flags & GGML_TENSOR_FLAG_OUTPUT);
    }

    // the node (after i) consuming t, if t has exactly one consumer
    const ggml_tensor * sole_consumer(const ggml_tensor * t, int from) const {
        if (!single_use(t)) return nullptr;
        for (int j = from; j < cg->n_nodes; j++) {
            for (int s = 0; s < GGML_MAX_SRC; s++) {
                if (cg->nodes[j]->src[s] == t) return cg->nodes[j];
            }
        }
        return nullptr;
    }

    // the quantized weight type shared by every consumer of t after node
    // `from`, when all of them are MUL_MATs reading t as activations; else -1
    int quant_consumers(const ggml_tensor * t, int from) const {
        int wt = -1;
        for (int j = from; j < cg->n_nodes; j++) {
            const ggml_tensor * c = cg->nodes[j];
            bool reads = false;
            for (int s = 0; s < GGML_MAX_SRC; s++) reads = reads || c->src[s] == t;
            if (!reads) continue;
            if (c->op != GGML_OP_MUL_MAT || c->src[1] != t || c->src[0] == t) return -1;
            const int w = c->src[0]->type;
            if ((w != GGML_TYPE_Q8_0 && w != GGML_TYPE_Q4_K) || c->src[0]->ne[0] != t->ne[0] ||
                !supports_op(be->dev, c))
                return -1;
            if (wt >= 0 && w != wt) return -1;
            wt = w;
        }
        return wt;
    }

    // a launch at the current position writing `writes` (default: the bytes of `node`)
    // (a list holding only nullptr: the step writes no graph tensor, only scratch)
    void add_step(std::function<void(hipStream_t)> fn, const ggml_tensor * node, const char * label,
                  std::vector<const ggml_tensor *> writes = {}) {
        step s;
        s.run = std::move(fn);
        s.node = node;
        s.label = label;
        s.pos = cur;
        if (writes.size() == 0) writes = {node};
        for (const ggml_tensor * w : writes) {
            const span sp = span_of(w);
            if (sp.lo < sp.hi) s.writes.push_back({sp.lo, sp.hi});
        }
        if (plan_trace()) {
            std::fprintf(stderr, "mi355x plan: step %zu at node %d %s", steps.size(), cur, label);
            for (const ggml_tensor * w : writes)
                if (w) std::fprintf(stderr, " [%s %s]", ggml_op_name(w->op), w->name);
            std::fprintf(stderr, "\n");
        }
        steps.push_back(std::move(s));
    }
    // OPENASR_MI355X_PLAN_TRACE=1: each planned launch on stderr (its label,
    // the graph position it runs at, the nodes it writes)
    static bool plan_trace() {
        static const bool on = [] {
            const char * e = std::getenv("OPENASR_MI355X_PLAN_TRACE");
            return e && e[0] == '1';
        }();
        return on;
    }

    bool validate();

    bool fail(const ggml_tensor * t, const char * why) {
        char buf[256];
        std::snprintf(buf, sizeof(buf), "node '%s' (op %d): %s", t->name, (int) t->op, why);
        error = buf;
        return false;
    }

    // norms whose launch is skipped: the GEMVs consuming their output
    // normalise and quantize in their activation prologue (norm output -> it)
    std::unordered_map<const ggml_tensor *, gemv_prologue> pro_norm;
    std::unordered_map<const ggml_tensor *, span> pro_norm_in;  // the bytes such a prologue reads

    // the rope table the scratch holds at this point of the plan
    struct rope_key {
        const int32_t * pos = nullptr;
        int n_seq = 0;
        float theta_scale = 0, freq_scale = 0, attn_factor = 0;
    } rope_cur;

    // at most this many 16-row tiles take a prologue: every workgroup stages
    // the activations itself, so the redundant staging grows with the grid
    static constexpr int64_t kProMaxTiles = 512;

    static bool use_mmq(int wtype, int64_t M, int64_t K, int64_t N) {
        return mmq_supported(wtype, M, K) && N > 16 && (N > 64 || M >= 8192);
    }

    // the MUL_MAT c (quantized weights, activations of K x N) runs as an MFMA
    // GEMV that can take an activation prologue
    bool prologue_gemv(const ggml_tensor * c, bool norm) const {
        const ggml_tensor * w = c->src[0];
        const int64_t K = w->ne[0], M = w->ne[1];
        const int64_t N = c->src[1]->ne[1] * c->src[1]->ne[2] * c->src[1]->ne[3];
        return !use_mmq(w->type, M, K, N) && gemv_mfma_supported(w->type, M, K) && M / 16 <= kProMaxTiles &&
               gemv_prologue_supported(w->type, M, K, N, norm);
    }

    static bool aligned16(const void * p) { return ((uintptr_t) p & 15) == 0; }

    // an f32 view whose columns the prologue can read: unit stride, columns
    // at a uniform 16-byte-aligned stride
    static bool prologue_view(const tview & v) {
        if (v.nb[0] != 4 || !aligned16(v.data) || v.nb[1] % 16 != 0) return false;
        if (v.ne[2] > 1 && v.nb[2] != v.nb[1] * v.ne[1]) return false;
        if (v.ne[3] > 1 && v.nb[3] != v.nb[2] * v.ne[2]) return false;
        return true;
    }

    // bytes [lo, hi) a view spans
    static void view_span(const tview & v, int64_t elem, uintptr_t & lo, uintptr_t & hi) {
        int64_t last = elem;
        for (int d = 0; d < 4; d++) last += (v.ne[d] - 1) * v.nb[d];
        lo = (uintptr_t) v.data;
        hi = lo + (uintptr_t) last;
    }

    // no node between positions i and j (inclusive) that may run writes into
    // the bytes of view v
    bool untouched_until(const tview & v, int i, int j) const {
        uintptr_t lo, hi;
        view_span(v, 4, lo, hi);
        for (int k = i + 1; k <= j && k < cg->n_nodes; k++) {
            const ggml_tensor * n = cg->nodes[k];
            if (is_view_op(n->op) || n->op == GGML_OP_NONE || !n->data) continue;
            const uintptr_t a = (uintptr_t) n->data, b = a + ggml_nbytes(n);
            if (a < hi && lo < b) return false;
        }
        return true;
    }

    bool plan();
    bool plan_mul_mat(int i, const ggml_tensor * t);
    bool hoist_ok(int i, const hoist & h) const;
    // t is available before node i runs: a leaf, or a node planned earlier
    bool ready_before(const ggml_tensor * t, int i) const {
        while (t->view_src) t = t->view_src;
        auto it = index.find(t);
        return it == index.end() || it->second < i;
    }
    bool plan_norm(int i, const ggml_tensor * t);
    bool norm_rope_match(int i, const ggml_tensor * t, norm_rope_job & job, const ggml_tensor *& mul,
                         const ggml_tensor *& rope) const;
    bool plan_unary(int i, const ggml_tensor * t);
    bool plan_binary(const ggml_tensor * t);
    bool plan_fattn(int i, const ggml_tensor * t);
    bool make_fattn(const ggml_tensor * t, fattn_args & a);
    void fattn_quant_out(int i, const ggml_tensor * t, fattn_args & a, const ggml_tensor *& view);
    bool plan_attn_step(int i, const ggml_tensor * t);
};

// The unfused attention chains of the graph (llm_naive_masked_attention,
// nn/decoder.rs:2154-2200): SOFT_MAX_EXT P over S = MUL_MAT(K, Q), read only
// by C = MUL_MAT(CONT(TRANSPOSE(V)), P), read only through PERMUTE(0, 2, 1, 3)
// by the output CONT O; K and V f16 rows (the caches, or their GQA
// expansions), Q f32. Each becomes one k_attn_naive launch at O.
void planner::find_naive() {
    for (int iP = 0; iP < cg->n_nodes; iP++) {
        const ggml_tensor * P = cg->nodes[iP];
        if (P->op != GGML_OP_SOFT_MAX || P->type != GGML_TYPE_F32 || op_f32(P, 1) != 0.0f) continue;
        const ggml_tensor *S = P->src[0], *M = P->src[1];
        if (!S || S->op != GGML_OP_MUL_MAT || !single_use(S) || !single_use(P)) continue;
        const ggml_tensor *Kx = S->src[0], *Q = S->src[1];
        if (Kx->type != GGML_TYPE_F16 || Q->type != GGML_TYPE_F32 || Q->nb[0] != 4) continue;
        const ggml_tensor * C = sole_consumer(P, iP + 1);
        if (!C || C->op != GGML_OP_MUL_MAT || C->src[1] != P || C->type != GGML_TYPE_F32 || !single_use(C)) continue;
        const ggml_tensor * VT = C->src[0];
        if (VT->op != GGML_OP_CONT || VT->type != GGML_TYPE_F16 || !single_use(VT) || !is_contiguous(VT)) continue;
        const ggml_tensor * TR = VT->src[0];
        if (TR->op != GGML_OP_TRANSPOSE || !single_use(TR)) continue;
        const ggml_tensor * Vx = TR->src[0];
        if (Vx->type != GGML_TYPE_F16) continue;
        const ggml_tensor * PM = sole_consumer(C, index.at(C) + 1);
        if (!PM || PM->op != GGML_OP_PERMUTE || !single_use(PM)) continue;
        const ggml_tensor * O = sole_consumer(PM, index.at(PM) + 1);
        if (!O || O->op != GGML_OP_CONT || O->type != GGML_TYPE_F32 || !is_contiguous(O) || no_naive.count(O)) continue;
        if ((S->flags | P->flags | VT->flags | C->flags) & GGML_TENSOR_FLAG_OUTPUT) continue;
        const int64_t D = Q->ne[0], nq = Q->ne[1], Hq = Q->ne[2], ns = Q->ne[3];
        // K and V as the launch reads them: the source of a GQA expansion
        // (query head h reads kv head h / g), or the operand itself
        tview kv = make_view(Kx), vv = make_view(Vx);
        const ggml_tensor *rk = nullptr, *rv = nullptr;
        tview fk, fv;
        const bool kf = match_gqa(Kx, rk, fk) && !no_fold.count(rk);
        const bool vf = match_gqa(Vx, rv, fv) && !no_fold.count(rv);
        if (kf != vf) continue;
        if (kf) kv = fk, vv = fv;
        const int64_t T = kv.ne[1], Hk = kv.ne[2];
        bool ok = kv.ne[0] == D && vv.ne[0] == D && vv.ne[1] == T && vv.ne[2] == Hk && vv.ne[3] == kv.ne[3] &&
                  kv.nb[0] == 2 && vv.nb[0] == 2 && Hk > 0 && Hq % Hk == 0 && kv.ne[3] > 0 && ns % kv.ne[3] == 0;
        ok = ok && S->ne[0] == T && S->ne[1] == nq && S->ne[2] == Hq && S->ne[3] == ns;
        ok = ok && C->ne[0] == D && C->ne[1] == nq && C->ne[2] == Hq && C->ne[3] == ns;
        ok = ok && TR->ne[0] == Vx->ne[1] && TR->ne[1] == Vx->ne[0] && TR->nb[0] == Vx->nb[1] && TR->nb[1] == Vx->nb[0];
        ok = ok && PM->ne[0] == D && PM->ne[1] == Hq && PM->ne[2] == nq && PM->ne[3] == ns && PM->nb[0] == C->nb[0] &&
             PM->nb[1] == C->nb[2] && PM->nb[2] == C->nb[1] && PM->nb[3] == C->nb[3] && PM->data == C->data;
        for (int d = 0; d < 4 && ok; d++) ok = O->ne[d] == PM->ne[d];
        ok = ok && ((uintptr_t) kv.data % 16 == 0) && kv.nb[1] % 16 == 0 && ((uintptr_t) vv.data % 16 == 0) &&
             vv.nb[1] % 16 == 0 && attn_naive_supported((int) D, (int) Hq, (int) Hk, T);
        if (M) ok = ok && M->type == GGML_TYPE_F16 && M->ne[0] >= T && M->ne[1] >= nq && M->nb[0] == 2;
        if (!ok) continue;
        naive_job j;
        j.S = S, j.P = P, j.VT = VT, j.C = C, j.O = O;
        naive_attn_args & a = j.a;
        a.q = (const char *) Q->data;
        a.q_nb1 = Q->nb[1], a.q_nb2 = Q->nb[2], a.q_nb3 = Q->nb[3];
        a.k = kv.data;
        a.k_nb1 = kv.nb[1], a.k_nb2 = kv.nb[2], a.k_nb3 = kv.nb[3];
        a.v = vv.data;
        a.v_nb1 = vv.nb[1], a.v_nb2 = vv.nb[2], a.v_nb3 = vv.nb[3];
        a.mask = M ? (const char *) M->data : nullptr;
        if (M) {
            a.m_nb1 = M->nb[1], a.m_nb2 = M->nb[2], a.m_nb3 = M->nb[3];
            a.m_ne2 = (int) M->ne[2], a.m_ne3 = (int) M->ne[3];
        } else {
            a.m_ne2 = a.m_ne3 = 1;
        }
        a.d = (int) D, a.hq = (int) Hq, a.hkv = (int) Hk, a.n_q = (int) nq, a.n_kv = (int) T, a.n_seq = (int) ns;
        a.rk3 = (int) (ns / kv.ne[3]);
        a.scale = op_f32(P, 0);
        a.q_f32 = S->op_params[0] == GGML_PREC_F32;
        a.p_f32 = C->op_params[0] == GGML_PREC_F32;
        a.out = (float *) O->data;
        // what the launch at O reads, and where the graph read it
        j.reads.push_back({span_of(kv, 2), index.at(S)});
        j.reads.push_back({span_of(make_view(Q), 4), index.at(S)});
        j.reads.push_back({span_of(vv, 2), index.at(VT)});
        if (M) j.reads.push_back({span_of(M), index.at(P)});
        naive_jobs[O] = j;
        for (const ggml_tensor * n : {S, P, VT, C}) naive_nodes.insert(n);
    }
}

// REPEATs every reader of which folds them (match_gqa): a FLASH_ATTN_EXT's
// K or V, or a fused attention chain's scores product and V^T copy. Their
// readers read the source instead, so the REPEAT is not launched.
void planner::find_gqa_skip() {
    for (int i = 0; i < cg->n_nodes; i++) {
        const ggml_tensor * r = cg->nodes[i];
        if (r->op != GGML_OP_REPEAT || no_fold.count(r) || (r->flags & GGML_TENSOR_FLAG_OUTPUT)) continue;
        bool ok = true, any = false;
        for (int j = i + 1; j < cg->n_nodes && ok; j++) {
            const ggml_tensor * n = cg->nodes[j];
            if (is_view_op(n->op)) continue;
            for (int k = 0; k < GGML_MAX_SRC && ok; k++) {
                const ggml_tensor * x = n->src[k];
                if (!x || root_of(x) != r) continue;
                any = true;
                const ggml_tensor * rr = nullptr;
                tview v;
                const bool fold = match_gqa(x, rr, v);
                if (n->op == GGML_OP_FLASH_ATTN_EXT && (k == 1 || k == 2) && fold && x->type == GGML_TYPE_F16) continue;
                if (naive_nodes.count(n) && ((n->op == GGML_OP_MUL_MAT && k == 0 && fold) || n->op == GGML_OP_CONT)) continue;
                ok = false;
            }
        }
        if (ok && any) {
            gqa_skip.insert(r);
            // the readers read the source where the REPEAT read it
            int last = i;
            for (int j = i + 1; j < cg->n_nodes; j++) {
                for (int k = 0; k < GGML_MAX_SRC; k++)
                    if (cg->nodes[j]->src[k] && root_of(cg->nodes[j]->src[k]) == r) last = j;
            }
            fold_reads.push_back({r, span_of(r->src[0]), i, last});
        }
    }
    // a fused chain whose K / V expansion is still launched reads the
    // expanded operands; if only one of the two folds, the chain runs op by op
    for (auto it = naive_jobs.begin(); it != naive_jobs.end();) {
        const naive_job & j = it->second;
        const ggml_tensor * Vx = j.VT->src[0]->src[0];
        tview fk, fv;
        const bool kf = gqa_fold(j.S->src[0], fk), vf = gqa_fold(Vx, fv);
        const ggml_tensor *rk = nullptr, *rv = nullptr;
        tview t0;
        const bool kr = match_gqa(j.S->src[0], rk, t0), vr = match_gqa(Vx, rv, t0);
        if (kf == kr && vf == vr) {
            ++it;
            continue;
        }
        for (const ggml_tensor * n : {j.S, j.P, j.VT, j.C}) naive_nodes.erase(n);
        no_naive.insert(it->first);
        naive_dropped = true;
        it = naive_jobs.erase(it);
    }
}

// May the launch at position i do the work described by h? Its own writes// May the launch at position i do the work described by h? Its own writes
// must not overlap what it reads (other workgroups of the launch may still
// be reading), except an exact in-place residual, nor each other; and every
// node between i and the last node it absorbs, which now runs after the
// launch although it ran before some of that work, must neither read what the
// launch writes nor write what it reads or writes. A node whose evaluation is
// deferred into a consumer is taken to read its sources too.
bool planner::hoist_ok(int i, const hoist & h) const {
    auto exact_inplace = [&](span w, span r) {
        for (const auto & pr : h.inplace) {
            const span a = span_of(pr.first), b = span_of(pr.second);
            if (a.lo == w.lo && a.hi == w.hi && b.lo == r.lo && b.hi == r.hi && a.lo == b.lo &&
                pr.first->nb[1] == pr.second->nb[1] && pr.first->nb[2] == pr.second->nb[2] &&
                pr.first->nb[3] == pr.second->nb[3])
                return true;
        }
        return false;
    };
    for (size_t a = 0; a < h.writes.size(); a++) {
        for (const span & r : h.reads)
            if (overlap(h.writes[a], r) && !exact_inplace(h.writes[a], r)) return false;
        for (size_t b = a + 1; b < h.writes.size(); b++)
            if (overlap(h.writes[a], h.writes[b])) return false;
    }
    int jmax = i;
    for (const ggml_tensor * n : h.nodes) {
        auto it = index.find(n);
        if (it != index.end()) jmax = std::max(jmax, it->second);
    }
    auto absorbed = [&](const ggml_tensor * n) {
        for (const ggml_tensor * x : h.nodes)
            if (x == n) return true;
        return false;
    };
    auto reads_written = [&](const ggml_tensor * x) {
        const span sx = span_of(x);
        for (const span & w : h.writes)
            if (overlap(sx, w)) return true;
        return false;
    };
    for (int k = i + 1; k <= jmax && k < cg->n_nodes; k++) {
        const ggml_tensor * n = cg->nodes[k];
        if (is_view_op(n->op) || absorbed(n)) continue;
        const span nw = span_of(n);
        for (const span & r : h.reads)
            if (overlap(nw, r)) return false;
        for (const span & w : h.writes)
            if (overlap(nw, w)) return false;
        for (int q = 0; q < GGML_MAX_SRC; q++) {
            const ggml_tensor * x = n->src[q];
            if (!x) continue;
            if (reads_written(x)) return false;
            if (deferred.count(x) || deferred.count(root_of(x))) {
                const ggml_tensor * d = deferred.count(x) ? x : root_of(x);
                for (int q2 = 0; q2 < GGML_MAX_SRC; q2++)
                    if (d->src[q2] && reads_written(d->src[q2])) return false;
            }
        }
    }
    return true;
}

bool planner::plan_mul_mat(int i, const ggml_tensor * t) {
    const ggml_tensor * w = t->src[0];
    const ggml_tensor * x = t->src[1];
    const tview xv = make_view(x);
    if (w->type == GGML_TYPE_Q3_K) {
        // Q3_K weights (the host's q3_k pack policy, pack_quant.rs:205-207):
        // the columns quantized to Q8_K as for Q4_K, then the row-team GEMV
        // (eight columns a launch), exact block sums; no folds
        const int64_t K = w->ne[0], M = w->ne[1];
        const int64_t N = x->ne[1] * x->ne[2] * x->ne[3];
        const char * W = (const char *) w->data;
        const int64_t row_bytes = (int64_t) w->nb[1];
        act_need = std::max(act_need, act_bytes(GGML_TYPE_Q3_K, K, N));
        const bool reuse = act_src == x && act_wtype == GGML_TYPE_Q3_K;
        if (!reuse && reads_unwritten(t, x)) return false;
        hoist h;
        h.reads.push_back(span_of(w));
        h.writes.push_back(span_of(t));
        if (!hoist_ok(i, h)) return fail(t, "MUL_MAT output overlaps its own input");
        act_src = x;
        act_wtype = GGML_TYPE_Q3_K;
        backend_state * b = be;
        const int ncu = n_cu;
        char * dst = (char *) t->data;
        const int64_t dst_nb1 = (int64_t) t->nb[1];
        if (!reuse) {
            add_step(
                [=](hipStream_t s) {
                    act_buffers act = act_carve(GGML_TYPE_Q3_K, act_base(b), K, N);
                    launch_quantize_act(xv, GGML_TYPE_Q3_K, act, s);
                },
                t, "quantize_q8_K", {nullptr});
        }
        add_step(
            [=](hipStream_t s) {
                act_buffers act = act_carve(GGML_TYPE_Q3_K, act_base(b), K, N);
                launch_mmv(GGML_TYPE_Q3_K, W, row_bytes, M, K, act, N, dst, dst_nb1, s, ncu);
            },
            t, "mul_mat_q3_K");
        return true;
    }
    if (w->type == GGML_TYPE_Q8_0 || w->type == GGML_TYPE_Q4_K) {
        const int wtype = w->type;
        const int64_t K = w->ne[0], M = w->ne[1];
        const int64_t N = x->ne[1] * x->ne[2] * x->ne[3];
        const char * W = (const char *) w->data;
        const int64_t row_bytes = (int64_t) w->nb[1];
        act_need = std::max(act_need, act_bytes(wtype, K, N));
        const bool reuse = act_src == x && act_wtype == wtype;
        if (!reuse && reads_unwritten(t, x)) return false;
        backend_state * b = be;
        const int ncu = n_cu;
        // the tile GEMM once the columns outgrow a few GEMV chunks (earlier for tall matrices)
        const bool wide = use_mmq(wtype, M, K, N);
        const bool mfma = !wide && gemv_mfma_supported(wtype, M, K);
        // activation prologue: the norm in front (planned by plan_norm), or
        // the quantization of f32 activations no earlier step quantized
        bool has_pro = false;
        gemv_prologue pro;
        span pro_in;  // the f32 activations the prologue reads
        auto pn = pro_norm.find(x);
        if (pn != pro_norm.end()) {
            if (!mfma || !prologue_gemv(t, true)) return fail(t, "normalising prologue on a launch that cannot take it");
            pro = pn->second;
            has_pro = true;
            pro_in = pro_norm_in[x];
        } else if (!reuse && mfma && x->type == GGML_TYPE_F32 && prologue_view(xv) && prologue_gemv(t, false)) {
            pro.x = (const float *) xv.data;
            pro.x_nb1 = xv.nb[1];
            has_pro = true;
            pro_in = span_of(xv, 4);
        }
        if (!has_pro) {
            // the act region now holds x's quantization
            act_src = x;
            act_wtype = wtype;
        }
        // what the plain launch reads and writes; each fold below is taken
        // only if the launch with it still passes hoist_ok
        hoist h;
        h.reads.push_back(span_of(w));
        if (has_pro) h.reads.push_back(pro_in);
        h.writes.push_back(span_of(t));
        if (!hoist_ok(i, h)) return fail(t, "MUL_MAT output overlaps its own input");
        char * dst = (char *) t->data;
        int64_t dst_nb1 = (int64_t) t->nb[1];
        const ggml_tensor * produced = t;  // the last node the GEMV step writes
        // the launch writing `out` instead of `produced`, absorbing `nodes`
        // and reading `extra` (in place of `inplace_with`, if given)
        auto try_fold = [&](std::initializer_list<const ggml_tensor *> nodes, const ggml_tensor * out,
                            std::initializer_list<const ggml_tensor *> extra, const ggml_tensor * inplace_with) {
            hoist h2 = h;
            for (const ggml_tensor * n : nodes) h2.nodes.push_back(n);
            h2.writes[0] = span_of(out);
            for (const ggml_tensor * e : extra) h2.reads.push_back(span_of(e));
            if (inplace_with) h2.inplace.push_back({out, inplace_with});
            if (!hoist_ok(i, h2)) return false;
            h = h2;
            return true;
        };
        // the default precision (the graph's contract, op_params[0]) with
        // enough tiles and 16-byte weight rows: the f16 matrix-core form
        // (k_mmq_f16.hip, float tolerance)
        const bool mmq16_ok = wide && t->op_params[0] != GGML_PREC_F32 && mmq_f16_supported(wtype, M, K, N, n_cu) &&
                              row_bytes % 16 == 0 && aligned16(W);
        // SwiGLU: MUL_MAT(gate, x) -> SILU -> MUL with MUL_MAT(up, x) of the
        // same shape becomes one launch over both matrices (the GEMV, or the
        // f16 tile GEMM for 64-row multiples)
        const char * W2 = nullptr;
        const ggml_tensor * silu = mfma || (mmq16_ok && M % 64 == 0) ? sole_consumer(t, i + 1) : nullptr;
        if (silu && silu->op == GGML_OP_UNARY && silu->op_params[0] == GGML_UNARY_OP_SILU && silu->src[0] == t) {
            const ggml_tensor * hm = sole_consumer(silu, i + 1);
            const ggml_tensor * u = nullptr;
            if (hm && hm->op == GGML_OP_MUL && (hm->src[0] == silu || hm->src[1] == silu)) {
                u = hm->src[0] == silu ? hm->src[1] : hm->src[0];
            }
            bool ok = u && u->op == GGML_OP_MUL_MAT && u->src[1] == x && u->src[0]->type == wtype &&
                      u->src[0]->ne[0] == K && u->src[0]->ne[1] == M && u->src[0]->nb[1] == w->nb[1] &&
                      sole_consumer(u, i + 1) == hm && supports_op(be->dev, u) && is_contiguous(hm) &&
                      ready_before(u->src[0], i) && u->op_params[0] == t->op_params[0] &&
                      (mfma || aligned16(u->src[0]->data));
            for (int d = 0; d < 4 && ok; d++) ok = hm->ne[d] == t->ne[d] && u->ne[d] == t->ne[d];
            if (ok && try_fold({silu, u, hm}, hm, {u->src[0]}, nullptr)) {
                W2 = (const char *) u->src[0]->data;
                dst = (char *) hm->data;
                dst_nb1 = (int64_t) hm->nb[1];
                produced = hm;
            }
        }
        // the tile GEMM: a bias ADD (a row of the output's width), a residual
        // ADD of the output's shape and a GELU_ERF fold into its epilogue,
        // with the roundings of the separate ops
        gemm_float_epi mepi;
        if (wide && !W2 && is_contiguous(t)) {
            auto plain = [](const ggml_tensor * o) { return o->type == GGML_TYPE_F32 && is_contiguous(o); };
            auto shaped = [&](const ggml_tensor * o) {
                for (int d = 0; d < 4; d++)
                    if (o->ne[d] != t->ne[d]) return false;
                return true;
            };
            const ggml_tensor * add = sole_consumer(t, i + 1);
            if (add && add->op == GGML_OP_ADD && plain(add) && shaped(add)) {
                const ggml_tensor * o = add->src[0] == t ? add->src[1] : add->src[0];
                const bool row = o != t && plain(o) && o->ne[0] == t->ne[0] && o->ne[1] * o->ne[2] * o->ne[3] == 1;
                const bool full = o != t && plain(o) && shaped(o);
                if (row && ready_before(o, i) && try_fold({add}, add, {o}, nullptr)) {
                    mepi.bias = (const float *) o->data;
                    produced = add;
                } else if (full && ready_before(o, i) && try_fold({add}, add, {o}, o)) {
                    mepi.res = (const float *) o->data;
                    produced = add;
                }
            }
            const ggml_tensor * nx = produced != t ? sole_consumer(produced, i + 1) : nullptr;
            if (mepi.bias && nx && nx->op == GGML_OP_ADD && plain(nx) && shaped(nx)) {
                const ggml_tensor * r = nx->src[0] == produced ? nx->src[1] : nx->src[0];
                if (r != produced && plain(r) && shaped(r) && ready_before(r, i) && try_fold({nx}, nx, {r}, r)) {
                    mepi.res = (const float *) r->data;
                    produced = nx;
                }
            }
            const ggml_tensor * u = sole_consumer(produced, i + 1);
            if (u && u->op == GGML_OP_UNARY && u->op_params[0] == GGML_UNARY_OP_GELU_ERF && u->src[0] == produced &&
                plain(u) && shaped(u) && try_fold({u}, u, {}, nullptr)) {
                mepi.gelu_erf = true;
                produced = u;
            }
            dst = (char *) produced->data;
            dst_nb1 = (int64_t) produced->nb[1];
        }
        // sibling MUL_MATs of the same activations (an encoder block's q, k, v
        // projections, each maybe with a bias ADD) join the tile GEMM launch
        // as further row ranges; each is taken only if the launch with it
        // passes hoist_ok
        std::vector<gemm_float_sub> msubs;
        std::vector<const ggml_tensor *> msub_outs;
        if (wide && !W2 && is_contiguous(t) && !mepi.res && !mepi.gelu_erf && M % 64 == 0 && N == t->ne[1]) {
            for (int j = i + 1; j < cg->n_nodes && j <= i + 16 && (int) msubs.size() < kGemmFloatMaxSubs; j++) {
                const ggml_tensor * u = cg->nodes[j];
                if (is_view_op(u->op) || deferred.count(u)) continue;
                const ggml_tensor * uw = u->src[0];
                const bool sibling = u->op == GGML_OP_MUL_MAT && u->src[1] == x && uw->type == wtype &&
                                     u->op_params[0] == t->op_params[0] &&
                                     uw->ne[0] == K && uw->ne[2] == 1 && uw->ne[3] == 1 &&
                                     (int64_t) uw->nb[1] == row_bytes && uw->ne[1] % 64 == 0 &&
                                     u->type == GGML_TYPE_F32 && is_contiguous(u) && u->ne[1] == N && u->ne[2] == 1 &&
                                     u->ne[3] == 1 && ready_before(uw, i);
                if (!sibling) continue;
                gemm_float_sub sb;
                sb.a = (const char *) uw->data;
                sb.M = uw->ne[1];
                sb.d = (char *) u->data;
                hoist h2 = h;
                h2.nodes.push_back(u);
                h2.reads.push_back(span_of(uw));
                const ggml_tensor * out = u;
                const ggml_tensor * ua = sole_consumer(u, j + 1);
                if (ua && ua->op == GGML_OP_ADD && ua->type == GGML_TYPE_F32 && is_contiguous(ua)) {
                    const ggml_tensor * o = ua->src[0] == u ? ua->src[1] : ua->src[0];
                    bool same = o != u;
                    for (int d = 0; d < 4 && same; d++) same = ua->ne[d] == u->ne[d];
                    const bool row = same && o->type == GGML_TYPE_F32 && is_contiguous(o) && o->ne[0] == u->ne[0] &&
                                     o->ne[1] * o->ne[2] * o->ne[3] == 1;
                    if (row && ready_before(o, i)) {
                        hoist h3 = h2;
                        h3.nodes.push_back(ua);
                        h3.reads.push_back(span_of(o));
                        h3.writes.push_back(span_of(ua));
                        if (hoist_ok(i, h3)) {
                            sb.bias = (const float *) o->data;
                            sb.d = (char *) ua->data;
                            out = ua;
                            h2 = h3;
                        }
                    }
                }
                if (out == u) {
                    h2.writes.push_back(span_of(u));
                    if (!hoist_ok(i, h2)) break;
                }
                h = h2;
                msubs.push_back(sb);
                msub_outs.push_back(out);
            }
        }
        bool mmq16 = mmq16_ok;
        for (const gemm_float_sub & sb : msubs) mmq16 = mmq16 && aligned16(sb.a);
        if (mmq16) gen_need = std::max(gen_need, mmq_f16_scratch_bytes(K, N));
        // a following residual ADD of the same shape folds into the epilogue
        const char * res = nullptr;
        int64_t res_nb1 = 0;
        const ggml_tensor * add = mfma && !W2 ? sole_consumer(t, i + 1) : nullptr;
        if (add && add->op == GGML_OP_ADD && add->type == GGML_TYPE_F32 && is_contiguous(add)) {
            const ggml_tensor * o = add->src[0] == t ? add->src[1] : add->src[0];
            bool same = o != t && o->type == GGML_TYPE_F32 && o->nb[0] == 4 && columns_foldable(o);
            for (int d = 0; d < 4 && same; d++) same = o->ne[d] == t->ne[d] && add->ne[d] == t->ne[d];
            if (same && ready_before(o, i) && try_fold({add}, add, {o}, o)) {
                res = (const char *) o->data;
                res_nb1 = (int64_t) o->nb[1];
                dst = (char *) add->data;
                dst_nb1 = (int64_t) add->nb[1];
                produced = add;
            }
        }
        // one column of Q8_0 weights: a second ADD (bias, then residual) or a
        // GELU after the first also folds into the single-column epilogue
        gemv_epilogue epi;
        if (res && mfma && gemv_single_column(wtype, K, N, has_pro && pro.norm >= 0)) {
            const ggml_tensor * nx = sole_consumer(produced, i + 1);
            if (nx && nx->op == GGML_OP_ADD && nx->type == GGML_TYPE_F32 && is_contiguous(nx)) {
                const ggml_tensor * o = nx->src[0] == produced ? nx->src[1] : nx->src[0];
                bool same = o != produced && o->type == GGML_TYPE_F32 && o->nb[0] == 4 && columns_foldable(o);
                for (int d = 0; d < 4 && same; d++) same = o->ne[d] == t->ne[d] && nx->ne[d] == t->ne[d];
                if (same && ready_before(o, i) && try_fold({nx}, nx, {o}, o)) {
                    epi.res2 = (const char *) o->data;
                    dst = (char *) nx->data;
                    produced = nx;
                }
            } else if (nx && nx->op == GGML_OP_UNARY && nx->op_params[0] == GGML_UNARY_OP_GELU &&
                       nx->src[0] == produced && nx->type == GGML_TYPE_F32 && is_contiguous(nx)) {
                bool same = true;
                for (int d = 0; d < 4 && same; d++) same = nx->ne[d] == t->ne[d];
                if (same && try_fold({nx}, nx, {}, nullptr)) {
                    epi.gelu = be->dev->gelu_table;
                    dst = (char *) nx->data;
                    produced = nx;
                }
            }
        }
        // sibling MUL_MATs of the same normalised column (Whisper's q, k, v
        // projections, each maybe with a bias ADD) join a one-column launch.
        // A sibling whose column only goes (through its RESHAPE to one row)
        // to a SET_ROWS into an f16 cache writes the cache row itself
        // (Whisper's self-attention K / V rows, the rounding of the separate
        // op) and not the f32 column. Each sibling is taken in the first of
        // these forms whose launch passes hoist_ok: bias and cache row, bias,
        // cache row, neither.
        std::vector<gemv_sub> subs;
        std::vector<const ggml_tensor *> sub_outs;  // the siblings' f32 columns the launch writes
        std::vector<const ggml_tensor *> row_outs;  // SET_ROWS the launch performs
        if (pn != pro_norm.end() && mfma && !W2 && !epi.res2 && !epi.gelu &&
            gemv_single_column(wtype, K, N, pro.norm >= 0)) {
            for (int j = i + 1; j < cg->n_nodes && j <= i + 16 && (int) subs.size() < kGemvMaxSubs; j++) {
                const ggml_tensor * u = cg->nodes[j];
                if (is_view_op(u->op) || deferred.count(u)) continue;
                const ggml_tensor * uw = u->src[0];
                const bool sibling = u->op == GGML_OP_MUL_MAT && u->src[1] == x && uw->type == wtype &&
                                     u->op_params[0] == t->op_params[0] &&
                                     uw->ne[0] == K && uw->ne[2] == 1 && uw->ne[3] == 1 &&
                                     (int64_t) uw->nb[1] == row_bytes && u->type == GGML_TYPE_F32 && is_contiguous(u) &&
                                     u->ne[1] * u->ne[2] * u->ne[3] == 1 && ready_before(uw, i);
                if (!sibling) continue;
                // the bias ADD (a tensor of the column's shape)
                const ggml_tensor * ua = sole_consumer(u, j + 1);
                const ggml_tensor * bias = nullptr;
                if (ua && ua->op == GGML_OP_ADD && ua->type == GGML_TYPE_F32 && is_contiguous(ua)) {
                    const ggml_tensor * o = ua->src[0] == u ? ua->src[1] : ua->src[0];
                    bool same = o != u && o->type == GGML_TYPE_F32 && o->nb[0] == 4 && columns_foldable(o);
                    for (int d = 0; d < 4 && same; d++) same = o->ne[d] == u->ne[d] && ua->ne[d] == u->ne[d];
                    if (same && ready_before(o, i)) bias = o;
                }
                // the cache row the column goes to
                auto set_rows_of = [&](const ggml_tensor * out) -> const ggml_tensor * {
                    const ggml_tensor * rs = sole_consumer(out, j + 1);
                    if (!rs || rs->op != GGML_OP_RESHAPE || rs->src[0] != out || rs->ne[0] != uw->ne[1] ||
                        rs->ne[1] != 1 || rs->ne[2] != 1 || rs->ne[3] != 1)
                        return nullptr;
                    const ggml_tensor * sr = sole_consumer(rs, j + 1);
                    if (!sr || sr->op != GGML_OP_SET_ROWS || sr->src[0] != rs || sr->type != GGML_TYPE_F16 ||
                        sr->nb[0] != 2 || sr->ne[0] != uw->ne[1] || sr->ne[2] != 1 || sr->ne[3] != 1)
                        return nullptr;
                    const ggml_tensor * ix = sr->src[1];
                    if (ggml_nelements(ix) != 1 || (ix->type != GGML_TYPE_I32 && ix->type != GGML_TYPE_I64) ||
                        !ready_before(ix, i) || !supports_op(be->dev, sr))
                        return nullptr;
                    return sr;
                };
                auto attempt = [&](bool with_bias, bool with_rows) {
                    const ggml_tensor * out = with_bias ? ua : u;
                    const ggml_tensor * sr = with_rows ? set_rows_of(out) : nullptr;
                    if ((with_bias && !bias) || (with_rows && !sr)) return false;
                    hoist h2 = h;
                    h2.nodes.push_back(u);
                    h2.reads.push_back(span_of(uw));
                    gemv_sub sb;
                    sb.W = (const char *) uw->data;
                    sb.M = uw->ne[1];
                    if (with_bias) {
                        h2.nodes.push_back(ua);
                        h2.reads.push_back(span_of(bias));
                        sb.res = (const char *) bias->data;
                    }
                    if (sr) {
                        h2.nodes.push_back(sr);
                        h2.reads.push_back(span_of(sr->src[1]));
                        h2.writes.push_back(span_of(sr));
                        sb.rows_dst = (char *) sr->data;
                        sb.rows_idx = (const char *) sr->src[1]->data;
                        sb.rows_i64 = sr->src[1]->type == GGML_TYPE_I64;
                        sb.rows_nb1 = (int64_t) sr->nb[1];
                        sb.rows_n = sr->ne[1];
                    } else {
                        h2.writes.push_back(span_of(out));
                        if (with_bias) h2.inplace.push_back({ua, bias});
                        sb.dst = (char *) out->data;
                    }
                    if (!hoist_ok(i, h2)) return false;
                    h = h2;
                    subs.push_back(sb);
                    if (sr) row_outs.push_back(sr);
                    else sub_outs.push_back(out);
                    return true;
                };
                if (!attempt(true, true) && !attempt(true, false) && !attempt(false, true) && !attempt(false, false)) break;
            }
        }
        for (const ggml_tensor * n : h.nodes) deferred[n] = n;
        std::vector<const ggml_tensor *> outs = {produced};
        outs.insert(outs.end(), sub_outs.begin(), sub_outs.end());
        outs.insert(outs.end(), msub_outs.begin(), msub_outs.end());
        outs.insert(outs.end(), row_outs.begin(), row_outs.end());
        if (!reuse && !has_pro) {
            add_step(
                [=](hipStream_t s) {
                    act_buffers act = act_carve(wtype, act_base(b), K, N);
                    launch_quantize_act(xv, wtype, act, s);
                },
                t, wtype == GGML_TYPE_Q8_0 ? "quantize_q8_0" : "quantize_q8_K", {nullptr});
        }
        add_step(
            [=](hipStream_t s) {
                act_buffers act = act_carve(wtype, act_base(b), K, N);
                if (mmq16)
                    launch_mmq_f16(wtype, W, row_bytes, M, K, act, N, dst, dst_nb1, gen_base(b), s, mepi,
                                   msubs.empty() ? nullptr : msubs.data(), (int) msubs.size(), W2);
                else if (wide)
                    launch_mmq(wtype, W, row_bytes, M, K, act, N, dst, dst_nb1, s, ncu, mepi,
                               msubs.empty() ? nullptr : msubs.data(), (int) msubs.size());
                else if (mfma)
                    launch_gemv_mfma(wtype, W, row_bytes, M, K, act, N, dst, dst_nb1, s, ncu, res, res_nb1, W2,
                                     has_pro ? &pro : nullptr, epi, subs.data(), (int) subs.size());
                else launch_mmv(wtype, W, row_bytes, M, K, act, N, dst, dst_nb1, s, ncu);
            },
            produced, W2 && mmq16 ? (wtype == GGML_TYPE_Q8_0 ? "mul_mat_swiglu_f16_q8_0" : "mul_mat_swiglu_f16_q4_K")
                      : W2      ? (wtype == GGML_TYPE_Q8_0 ? "mul_mat_swiglu_q8_0" : "mul_mat_swiglu_q4_K")
                      : mmq16   ? (wtype == GGML_TYPE_Q8_0 ? "mul_mat_f16_q8_0" : "mul_mat_f16_q4_K")
                              : (wtype == GGML_TYPE_Q8_0 ? "mul_mat_q8_0" : "mul_mat_q4_K"),
            outs);
        return true;
    }
    const tview dv = make_view(t);
    const tview wv = make_view(w);
    const int atype = w->type, btype = x->type;
    act_src = nullptr;
    // src0 an IM2COL result in the split layout (planned with it, see the
    // IM2COL case): only the bf16 form of this launch reads it
    const bool a_split = split_cols.count(root_of(w)) > 0;
    if (gemm_float_supported(dv, wv, atype, xv, btype)) {
        // the linear layers' bias ADD (a row of the output's width) and a
        // residual ADD of the output's shape fold into the epilogue, with
        // the two f32 roundings of the separate ops
        hoist h;
        h.reads.push_back(span_of(w));
        h.reads.push_back(span_of(xv, btype == GGML_TYPE_F16 ? 2 : 4));
        h.writes.push_back(span_of(t));
        if (!hoist_ok(i, h)) return fail(t, "MUL_MAT output overlaps its own input");
        const ggml_tensor * produced = t;
        gemm_float_epi epi;
        auto plain_f32 = [](const ggml_tensor * o) { return o->type == GGML_TYPE_F32 && is_contiguous(o); };
        auto try_fold = [&](const ggml_tensor * node, const ggml_tensor * o, bool inplace) {
            hoist h2 = h;
            h2.nodes.push_back(node);
            h2.writes[0] = span_of(node);
            h2.reads.push_back(span_of(o));
            if (inplace) h2.inplace.push_back({node, o});
            if (!hoist_ok(i, h2)) return false;
            h = h2;
            return true;
        };
        // a convolution's tail (ggml_conv_2d: the column GEMM's result
        // reshaped to [OW, OH, N, OC], PERMUTE(0, 1, 3, 2), CONT; then maybe
        // an ADD of one bias value a channel and GELU_ERF): the GEMM writes
        // the CONT's layout itself and adds the bias and the GELU in its
        // epilogue, the roundings of the separate ops
        const ggml_tensor * rs = sole_consumer(t, i + 1);
        const ggml_tensor * pm = rs && rs->op == GGML_OP_RESHAPE && rs->view_src == t ? sole_consumer(rs, i + 1) : nullptr;
        const ggml_tensor * ct = pm && pm->op == GGML_OP_PERMUTE && pm->src[0] == rs ? sole_consumer(pm, i + 1) : nullptr;
        if (ct && ct->op == GGML_OP_CONT && ct->src[0] == pm && plain_f32(t) && plain_f32(ct) && t->ne[2] == 1 &&
            t->ne[3] == 1) {
            const int64_t OW = rs->ne[0], OH = rs->ne[1], NB = rs->ne[2], OC = rs->ne[3];
            const bool perm = OW * OH * NB == t->ne[0] && OC == t->ne[1] && pm->ne[0] == OW && pm->ne[1] == OH &&
                              pm->ne[2] == OC && pm->ne[3] == NB && pm->nb[0] == 4 && pm->nb[1] == 4 * OW &&
                              pm->nb[2] == (size_t) t->nb[1] && pm->nb[3] == (size_t) (4 * OW * OH);
            hoist h2 = h;
            h2.nodes.push_back(ct);
            h2.writes[0] = span_of(ct);
            if (perm && hoist_ok(i, h2)) {
                h = h2;
                epi.perm_rows = OW * OH;
                produced = ct;
                const ggml_tensor * ad = sole_consumer(ct, i + 1);
                if (ad && ad->op == GGML_OP_ADD && plain_f32(ad) && ad->src[0] == ct) {
                    const ggml_tensor * b = ad->src[1];
                    bool shaped = true;
                    for (int d = 0; d < 4; d++) shaped = shaped && ad->ne[d] == ct->ne[d];
                    if (shaped && plain_f32(b) && b->ne[0] == 1 && b->ne[1] == 1 && b->ne[2] == OC && b->ne[3] == 1 &&
                        ready_before(b, i) && try_fold(ad, b, false)) {
                        epi.bias_col = (const float *) b->data;
                        produced = ad;
                    }
                }
                const ggml_tensor * ge = sole_consumer(produced, i + 1);
                if (ge && ge->op == GGML_OP_UNARY && ge->op_params[0] == GGML_UNARY_OP_GELU_ERF && ge->src[0] == produced &&
                    plain_f32(ge)) {
                    hoist h3 = h;
                    h3.nodes.push_back(ge);
                    h3.writes[0] = span_of(ge);
                    if (hoist_ok(i, h3)) {
                        h = h3;
                        epi.gelu_erf = true;
                        produced = ge;
                    }
                }
                for (const ggml_tensor * n : h.nodes) deferred[n] = n;
                tview ov = dv;
                ov.data = (char *) produced->data;
                const int splits = gemm_float_splits(dv, wv, atype, xv, btype, n_cu);
                gen_need = std::max(gen_need, gemm_float_split_bytes(dv, splits));
                backend_state * b = be;
                const bool x3 = t->op_params[0] != GGML_PREC_F32 && atype == GGML_TYPE_F32 && btype == GGML_TYPE_F32;
                add_step(
                    [=](hipStream_t s) {
                        launch_gemm_float(ov, wv, atype, xv, btype, s, epi, splits, (float *) gen_base(b), nullptr, 0,
                                          x3, a_split);
                    },
                    produced, atype == GGML_TYPE_F16 ? "conv_gemm_f16" : "conv_gemm_f32", {produced});
                return true;
            }
        }
        const ggml_tensor * add = sole_consumer(t, i + 1);
        if (add && add->op == GGML_OP_ADD && plain_f32(add) && is_contiguous(t)) {
            const ggml_tensor * o = add->src[0] == t ? add->src[1] : add->src[0];
            bool same = o != t;
            for (int d = 0; d < 4 && same; d++) same = add->ne[d] == t->ne[d];
            const bool row = same && plain_f32(o) && o->ne[0] == t->ne[0] && o->ne[1] * o->ne[2] * o->ne[3] == 1;
            if (row && ready_before(o, i) && try_fold(add, o, false)) {
                epi.bias = (const float *) o->data;
                produced = add;
                const ggml_tensor * add2 = sole_consumer(add, i + 1);
                if (add2 && add2->op == GGML_OP_ADD && plain_f32(add2)) {
                    const ggml_tensor * r = add2->src[0] == add ? add2->src[1] : add2->src[0];
                    bool same2 = r != add && plain_f32(r);
                    for (int d = 0; d < 4 && same2; d++) same2 = add2->ne[d] == t->ne[d] && r->ne[d] == t->ne[d];
                    if (same2 && ready_before(r, i) && try_fold(add2, r, true)) {
                        epi.res = (const float *) r->data;
                        produced = add2;
                    }
                }
            }
        }
        const ggml_tensor * ge = sole_consumer(produced, i + 1);
        if (ge && ge->op == GGML_OP_UNARY && ge->op_params[0] == GGML_UNARY_OP_GELU_ERF && ge->src[0] == produced &&
            plain_f32(ge) && is_contiguous(produced)) {
            bool same = true;
            for (int d = 0; d < 4 && same; d++) same = ge->ne[d] == t->ne[d];
            hoist h2 = h;
            h2.nodes.push_back(ge);
            h2.writes[0] = span_of(ge);
            if (same && hoist_ok(i, h2)) {
                h = h2;
                epi.gelu_erf = true;
                produced = ge;
            }
        }
        // sibling MUL_MATs of the same columns (an encoder block's q, k, v
        // projections, each maybe with a bias ADD) join the launch as further
        // row ranges; each is taken only if the launch with it passes hoist_ok
        std::vector<gemm_float_sub> subs;
        std::vector<const ggml_tensor *> sub_outs;
        if (!a_split && !epi.res && !epi.gelu_erf && gemm_float_siblings_ok(dv, wv, xv) && is_contiguous(t)) {
            for (int j = i + 1; j < cg->n_nodes && j <= i + 16 && (int) subs.size() < kGemmFloatMaxSubs; j++) {
                const ggml_tensor * u = cg->nodes[j];
                if (is_view_op(u->op) || deferred.count(u)) continue;
                const ggml_tensor * uw = u->src[0];
                const bool sibling = u->op == GGML_OP_MUL_MAT && u->src[1] == x && uw->type == w->type &&
                                     uw->ne[0] == w->ne[0] && uw->ne[2] == 1 && uw->ne[3] == 1 &&
                                     uw->nb[1] == w->nb[1] && uw->nb[0] == w->nb[0] && uw->ne[1] % 64 == 0 &&
                                     u->type == GGML_TYPE_F32 && is_contiguous(u) && u->ne[1] == t->ne[1] &&
                                     u->ne[2] == 1 && u->ne[3] == 1 && ready_before(uw, i) &&
                                     aligned16(uw->data);  // its rows take the same 16-byte loads
                if (!sibling) continue;
                gemm_float_sub sb;
                sb.a = (const char *) uw->data;
                sb.M = uw->ne[1];
                sb.d = (char *) u->data;
                hoist h2 = h;
                h2.nodes.push_back(u);
                h2.reads.push_back(span_of(uw));
                const ggml_tensor * out = u;
                const ggml_tensor * ua = sole_consumer(u, j + 1);
                if (ua && ua->op == GGML_OP_ADD && plain_f32(ua)) {
                    const ggml_tensor * o = ua->src[0] == u ? ua->src[1] : ua->src[0];
                    bool same = o != u;
                    for (int d = 0; d < 4 && same; d++) same = ua->ne[d] == u->ne[d];
                    const bool row = same && plain_f32(o) && o->ne[0] == u->ne[0] && o->ne[1] * o->ne[2] * o->ne[3] == 1;
                    if (row && ready_before(o, i)) {
                        hoist h3 = h2;
                        h3.nodes.push_back(ua);
                        h3.reads.push_back(span_of(o));
                        h3.writes.push_back(span_of(ua));
                        if (hoist_ok(i, h3)) {
                            sb.bias = (const float *) o->data;
                            sb.d = (char *) ua->data;
                            out = ua;
                            h2 = h3;
                        }
                    }
                }
                if (out == u) {
                    h2.writes.push_back(span_of(u));
                    if (!hoist_ok(i, h2)) break;
                }
                h = h2;
                subs.push_back(sb);
                sub_outs.push_back(out);
            }
        }
        for (const ggml_tensor * n : h.nodes) deferred[n] = n;
        tview ov = dv;
        ov.data = (char *) produced->data;
        // split K where the tiles leave CUs idle: partials in per-launch scratch
        const int splits = subs.empty() ? gemm_float_splits(dv, wv, atype, xv, btype, n_cu) : 1;
        gen_need = std::max(gen_need, gemm_float_split_bytes(dv, splits));
        backend_state * b = be;
        std::vector<const ggml_tensor *> outs = {produced};
        outs.insert(outs.end(), sub_outs.begin(), sub_outs.end());
        // F32 x F32 at the default precision (the graph's contract): the
        // bf16 hi / lo form on the matrix cores (float tolerance)
        const bool x3 = t->op_params[0] != GGML_PREC_F32 && atype == GGML_TYPE_F32 && btype == GGML_TYPE_F32;
        add_step(
            [=](hipStream_t s) {
                launch_gemm_float(ov, wv, atype, xv, btype, s, epi, splits, (float *) gen_base(b),
                                  subs.empty() ? nullptr : subs.data(), (int) subs.size(), x3, a_split);
            },
            produced, atype == GGML_TYPE_F16 ? "mul_mat_f16" : "mul_mat_f32", outs);
        return true;
    }
    if (a_split) return fail(t, "split column matrix outside its bf16 GEMM");
    if (btype != GGML_TYPE_F32) return fail(t, "f16 columns outside the matrix-core GEMM");
    add_step([=](hipStream_t s) { launch_mul_mat_float(dv, wv, atype, xv, s); }, t, "mul_mat_float");
    return true;
}

// RMS_NORM -> MUL(w) -> full-width NEOX ROPE over 128-element rows, the
// per-head QK-norm and rotary embedding of nn/decoder.rs:1937-1968: the job
// and the nodes it covers (mul, rope), or false
bool planner::norm_rope_match(int i, const ggml_tensor * t, norm_rope_job & job, const ggml_tensor *& mul,
                              const ggml_tensor *& rope) const {
    if (t->op != GGML_OP_RMS_NORM || t->ne[0] != 128 || !supports_op(be->dev, t)) return false;
    mul = sole_consumer(t, i + 1);
    if (!mul || mul->op != GGML_OP_MUL || mul->src[0] != t) return false;
    const ggml_tensor * wt = mul->src[1];
    if (wt->type != GGML_TYPE_F32 || wt->op != GGML_OP_NONE || !is_contiguous(wt) || wt->ne[0] != 128 ||
        wt->ne[1] != 1 || wt->ne[2] != 1 || wt->ne[3] != 1)
        return false;
    rope = sole_consumer(mul, i + 1);
    if (!rope || rope->op != GGML_OP_ROPE || rope->src[0] != mul || !supports_op(be->dev, rope) ||
        rope->op_params[2] != GGML_ROPE_TYPE_NEOX || rope->op_params[1] != 128 || rope->nb[0] != 4)
        return false;
    const tview av = view_of(t->src[0]);
    if (av.nb[0] != 4) return false;
    job = make_norm_rope_job(make_view(rope), av, op_f32(t, 0), (const float *) wt->data,
                             (const int32_t *) rope->src[1]->data, op_f32(rope, 5), op_f32(rope, 6), op_f32(rope, 8));
    return true;
}

bool planner::plan_norm(int i, const ggml_tensor * t) {
    if (plan_attn_step(i, t)) return true;
    {
        norm_rope_job j0, j1;
        const ggml_tensor *mul0, *rope0, *mul1, *rope1;
        if (norm_rope_match(i, t, j0, mul0, rope0)) {
            deferred[mul0] = mul0;
            deferred[rope0] = rope0;
            // the next planned node, if it is the same fusion over rows ready
            // now (the key rows after the query rows), shares the launch
            const ggml_tensor * t1 = nullptr;
            int i1 = -1;
            for (int j = i + 1; j < cg->n_nodes; j++) {
                const ggml_tensor * n = cg->nodes[j];
                if (is_view_op(n->op) || bypass.count(n) || deferred.count(n)) continue;
                t1 = n;
                i1 = j;
                break;
            }
            bool pair = t1 && norm_rope_match(i1, t1, j1, mul1, rope1);
            if (pair) {
                const ggml_tensor * src = root_of(t1->src[0]);
                auto bp = bypass.find(src);
                if (bp != bypass.end()) src = root_of(bp->second);
                pair = ready_before(src, i) && src != rope0 && src != mul0;
            }
            if (pair) {
                deferred[t1] = t1;
                deferred[mul1] = mul1;
                deferred[rope1] = rope1;
                add_step([=](hipStream_t s) { launch_rms_norm_rope128(j0, &j1, s); }, rope1, "rms_norm_rope",
                         {rope0, rope1});
            } else {
                add_step([=](hipStream_t s) { launch_rms_norm_rope128(j0, nullptr, s); }, rope0, "rms_norm_rope");
            }
            return true;
        }
    }
    const int mode = t->op == GGML_OP_RMS_NORM ? 0 : 1;
    const float eps = op_f32(t, 0);
    const ggml_tensor * out = t;
    const ggml_tensor * wt = nullptr;
    const ggml_tensor * bt = nullptr;
    // the fused kernel runs at the norm's position, so the weight and bias it
    // absorbs must already exist then: leaves (weights, inputs) only
    auto leaf = [](const ggml_tensor * x) {
        return x->op == GGML_OP_NONE || (is_view_op(x->op) && x->view_src && x->view_src->op == GGML_OP_NONE);
    };
    const ggml_tensor * mul = sole_consumer(t, i + 1);
    if (mul && mul->op == GGML_OP_MUL && mul->src[0] == t && mul->src[1]->type == GGML_TYPE_F32 &&
        mul->src[1]->ne[0] == t->ne[0] && leaf(mul->src[1])) {
        wt = mul->src[1];
        out = mul;
        deferred[mul] = mul;
        const ggml_tensor * add = sole_consumer(mul, i + 1);
        if (mode == 1 && add && add->op == GGML_OP_ADD && add->src[0] == mul && add->src[1]->type == GGML_TYPE_F32 &&
            add->src[1]->ne[0] == t->ne[0] && leaf(add->src[1])) {
            bt = add->src[1];
            out = add;
            deferred[add] = add;
        }
    }
    const tview dv = make_view(out), av = view_of(t->src[0]);
    const bool hw = wt != nullptr, hb = bt != nullptr;
    const tview wv = hw ? make_view(wt) : tview{}, bv = hb ? make_view(bt) : tview{};
    // when only quantized MUL_MATs read the result, the norm kernel also
    // writes their quantized activations (they then skip their quantize step)
    int qt = quant_consumers(out, i + 1);
    if (qt >= 0 && !(out->flags & GGML_TENSOR_FLAG_OUTPUT) && prologue_view(av) && av.ne[0] == out->ne[0] &&
        (!hw || aligned16(wt->data)) && (!hb || aligned16(bt->data))) {
        // every consumer a prologue GEMV, and the norm's input still intact
        // when the last of them runs
        bool ok = true;
        int last = i;
        for (int j = i + 1; j < cg->n_nodes && ok; j++) {
            const ggml_tensor * c = cg->nodes[j];
            if (c->op == GGML_OP_MUL_MAT && c->src[1] == out) {
                ok = prologue_gemv(c, true);
                last = j;
            }
        }
        if (ok && last > i && untouched_until(av, i, last)) {
            gemv_prologue p;
            p.x = (const float *) av.data;
            p.x_nb1 = av.nb[1];
            p.w = hw ? (const float *) wt->data : nullptr;
            p.b = hb ? (const float *) bt->data : nullptr;
            p.eps = eps;
            p.norm = mode;
            pro_norm[out] = p;
            pro_norm_in[out] = span_of(av, 4);
            return true;
        }
    }
    if (qt >= 0 && !norm_rows_supported(dv, av, hw ? &wv : nullptr, hb ? &bv : nullptr)) qt = -1;
    const int64_t K = out->ne[0], N = out->ne[1] * out->ne[2] * out->ne[3];
    if (qt >= 0) act_need = std::max(act_need, act_bytes(qt, K, N));
    backend_state * b = be;
    add_step(
        [=](hipStream_t s) {
            act_buffers ab{nullptr, nullptr, nullptr};
            if (qt >= 0) ab = act_carve(qt, act_base(b), K, N);
            launch_norm(dv, av, mode, eps, hw ? &wv : nullptr, hb ? &bv : nullptr, s, qt, qt >= 0 ? &ab : nullptr);
        },
        out, mode == 0 ? "rms_norm" : "norm");
    if (qt >= 0) {
        act_src = out;
        act_wtype = qt;
    }
    return true;
}

bool planner::plan_unary(int i, const ggml_tensor * t) {
    const int uop = t->op_params[0];
    const int ncu = n_cu;
    if (uop == GGML_UNARY_OP_SILU && !no_defer.count(t)) {
        const ggml_tensor * mul = sole_consumer(t, i + 1);
        if (mul && mul->op == GGML_OP_MUL && (mul->src[0] == t || mul->src[1] == t)) {
            const ggml_tensor * other = mul->src[0] == t ? mul->src[1] : mul->src[0];
            bool same_shape = true;
            for (int d = 0; d < 4; d++) same_shape = same_shape && other->ne[d] == mul->ne[d];
            if (same_shape) {
                // the SiLU is evaluated inside the multiply, at the multiply's position
                deferred[t] = mul;
                deferred_unary.push_back({t, index.at(mul)});
                return true;
            }
        }
    }
    const tview dv = make_view(t), av = make_view(t->src[0]);
    const uint16_t * gt = be->dev->gelu_table;
    add_step([=](hipStream_t s) { launch_unary(dv, av, uop, gt, s, ncu); }, t, "unary");
    return true;
}

bool planner::plan_binary(const ggml_tensor * t) {
    const int ncu = n_cu;
    // SiLU(gate) * up with the SiLU deferred into this node
    for (int k = 0; k < 2; k++) {
        const ggml_tensor * s = t->src[k];
        auto it = deferred.find(s);
        if (t->op == GGML_OP_MUL && s && s->op == GGML_OP_UNARY && it != deferred.end() && it->second == t) {
            const tview dv = make_view(t), gv = make_view(s->src[0]), uv = make_view(t->src[1 - k]);
            add_step([=](hipStream_t st) { launch_silu_mul(dv, gv, uv, st, ncu); }, t, "silu_mul");
            return true;
        }
    }
    const tview dv = make_view(t), av = view_of(t->src[0]), bv = view_of(t->src[1]);
    const int op = t->op;
    add_step([=](hipStream_t s) { launch_binary(op, dv, av, bv, s, ncu); }, t, "binary");
    return true;
}

bool planner::make_fattn(const ggml_tensor * t, fattn_args & a) {
    const ggml_tensor *q = t->src[0], *k = t->src[1], *v = t->src[2], *m = t->src[3];
    // K and V behind GQA expansions that are not launched: the sources'
    // kv heads (query head h reads head h / (hq / hkv), the kernel's rule)
    tview kv = make_view(k), vv = make_view(v);
    const bool kf = gqa_fold(k, kv), vf = gqa_fold(v, vv);
    if (kf != vf) return fail(t, "only one of K and V is a folded GQA expansion");
    a = fattn_args{};
    a.q = (const char *) q->data;
    a.k = kv.data;
    a.v = vv.data;
    a.mask = m ? (const char *) m->data : nullptr;
    a.q_nb1 = q->nb[1];
    a.q_nb2 = q->nb[2];
    a.q_nb3 = q->nb[3];
    a.k_nb1 = kv.nb[1];
    a.k_nb2 = kv.nb[2];
    a.k_nb3 = kv.nb[3];
    a.v_nb1 = vv.nb[1];
    a.v_nb2 = vv.nb[2];
    a.v_nb3 = vv.nb[3];
    if (m) {
        a.m_nb1 = m->nb[1];
        a.m_nb2 = m->nb[2];
        a.m_nb3 = m->nb[3];
        a.m_ne2 = (int) m->ne[2];
        a.m_ne3 = (int) m->ne[3];
        if (m->ne[0] < kv.ne[1] || m->ne[1] < q->ne[1]) return fail(t, "mask smaller than the attention span");
    }
    a.d = (int) q->ne[0];
    a.n_q = (int) q->ne[1];
    a.hq = (int) q->ne[2];
    a.n_seq = (int) q->ne[3];
    a.n_kv = (int) kv.ne[1];
    a.hkv = (int) kv.ne[2];
    if (a.hkv <= 0 || a.hq % a.hkv != 0 || vv.ne[2] != kv.ne[2] || vv.ne[1] != kv.ne[1])
        return fail(t, "K / V heads do not divide the query heads");
    a.rk3 = (int) (q->ne[3] / kv.ne[3]);
    a.scale = op_f32(t, 0);
    a.qtype = -1;
    // f16 K and V rows are read as 16-byte vectors (f32 ones are converted
    // into aligned scratch by plan_fattn)
    if ((k->type == GGML_TYPE_F16 && (uintptr_t) a.k % 16 != 0) || (v->type == GGML_TYPE_F16 && (uintptr_t) a.v % 16 != 0))
        return fail(t, "K/V not 16-byte aligned");
    fattn_plan(a, n_cu);
    // more than one query at the default precision (op_params[3], the
    // host's flash-attention precision contract): the matrix-core form
    a.mfma = t->op_params[3] != GGML_PREC_F32 && fattn_mfma_supported(a);
    if (a.mfma) fattn_mfma_plan(a, n_cu);
    // one query at the default precision: one workgroup per (sequence, kv
    // head, KV split), the waves merged in the launch (k_fattn_dec.hip),
    // where that form is the faster one
    if (!a.mfma && t->op_params[3] != GGML_PREC_F32 && fattn_dec_supported(a)) fattn_dec_plan(a, n_cu);
    if (!a.mfma && !a.dec && !fattn_fits(a)) return fail(t, "KV span longer than the kernel's chunk table");
    return true;
}

// the output projection consumes the output through a contiguous reshape:
// let the attention kernel quantize it for that MUL_MAT
void planner::fattn_quant_out(int i, const ggml_tensor * t, fattn_args & a, const ggml_tensor *& view) {
    const int g = a.hq / a.hkv;
    view = sole_consumer(t, i + 1);
    const ggml_tensor * mm = nullptr;
    if (view && (view->op == GGML_OP_RESHAPE || view->op == GGML_OP_VIEW) && view->view_src == t &&
        view->view_offs == 0 && is_contiguous(view) && view->ne[0] == (int64_t) a.d * a.hq) {
        mm = sole_consumer(view, i + 1);
    }
    if (mm && mm->op == GGML_OP_MUL_MAT && mm->src[1] == view && mm->src[0]->ne[0] == view->ne[0] &&
        supports_op(be->dev, mm)) {
        const int wt = mm->src[0]->type;
        if ((wt == GGML_TYPE_Q4_K && (g * a.d) % 256 == 0) || (wt == GGML_TYPE_Q8_0 && (g * a.d) % 32 == 0)) {
            a.qtype = wt;
            const int64_t K = view->ne[0], ncols = view->ne[1] * view->ne[2] * view->ne[3];
            act_need = std::max(act_need, act_bytes(wt, K, ncols));
            a.act = act_buffers{nullptr, nullptr, nullptr};
        }
    }
}

bool planner::plan_fattn(int i, const ggml_tensor * t) {
    fattn_args a;
    if (!make_fattn(t, a)) return false;
    const ggml_tensor * view = nullptr;
    if (!a.mfma) fattn_quant_out(i, t, a, view);
    // f32 K / V: rounded to contiguous f16 copies in scratch after the
    // partials -- the f16 definition over f16-rounded K / V, the conversion
    // ggml's GPU backends make as well
    const ggml_tensor *k = t->src[1], *v = t->src[2];
    const size_t part = (fattn_scratch_bytes(a) + 255) & ~(size_t) 255;
    const bool k32 = k->type == GGML_TYPE_F32, v32 = v->type == GGML_TYPE_F32;
    const size_t kbytes = k32 ? ((size_t) ggml_nelements(k) * 2 + 255) & ~(size_t) 255 : 0;
    const size_t vbytes = v32 ? ((size_t) ggml_nelements(v) * 2 + 255) & ~(size_t) 255 : 0;
    gen_need = std::max(gen_need, part + kbytes + vbytes);
    const tview kv = make_view(k), vv = make_view(v);
    backend_state * b = be;
    const int ncu = n_cu;
    float * out = (float *) t->data;
    const int64_t qK = (int64_t) a.d * a.hq, qN = (int64_t) a.n_q * a.n_seq;
    add_step(
        [=](hipStream_t s) {
            fattn_args la = a;
            if (la.qtype >= 0) la.act = act_carve(la.qtype, act_base(b), qK, qN);
            // contiguous f16 [ne0, ne1, ne2, ne3] copy of an f32 operand
            auto f16_dense = [](const tview & src, char * dst) {
                tview d = src;
                d.data = dst;
                d.nb[0] = 2;
                d.nb[1] = 2 * d.ne[0];
                d.nb[2] = d.nb[1] * d.ne[1];
                d.nb[3] = d.nb[2] * d.ne[2];
                return d;
            };
            auto dense_f32 = [](const tview & v) {
                return v.nb[0] == 4 && v.nb[1] == 4 * v.ne[0] && v.nb[2] == v.nb[1] * v.ne[1] &&
                       v.nb[3] == v.nb[2] * v.ne[2];
            };
            auto to_f16 = [&](const tview & src, char * dst, int64_t & nb1, int64_t & nb2, int64_t & nb3) {
                const tview d = f16_dense(src, dst);
                launch_copy(d, GGML_TYPE_F16, src, GGML_TYPE_F32, s, ncu);
                nb1 = d.nb[1];
                nb2 = d.nb[2];
                nb3 = d.nb[3];
            };
            char * g = gen_base(b);
            if (k32 && v32 && !dense_f32(kv) && !dense_f32(vv)) {
                // both strided head views: one launch for the two
                tview dk = f16_dense(kv, g + part), dvw = f16_dense(vv, g + part + kbytes);
                launch_copy_pair(dk, kv, dvw, vv, GGML_TYPE_F16, GGML_TYPE_F32, s, ncu);
                la.k = g + part, la.k_nb1 = dk.nb[1], la.k_nb2 = dk.nb[2], la.k_nb3 = dk.nb[3];
                la.v = g + part + kbytes, la.v_nb1 = dvw.nb[1], la.v_nb2 = dvw.nb[2], la.v_nb3 = dvw.nb[3];
            } else {
                if (k32) {
                    to_f16(kv, g + part, la.k_nb1, la.k_nb2, la.k_nb3);
                    la.k = g + part;
                }
                if (v32) {
                    to_f16(vv, g + part + kbytes, la.v_nb1, la.v_nb2, la.v_nb3);
                    la.v = g + part + kbytes;
                }
            }
            launch_fattn(la, g, out, s);
        },
        t, a.mfma ? "flash_attn_mfma" : a.dec ? "flash_attn_dec" : "flash_attn_ext");
    if (a.qtype >= 0) {
        act_src = view;
        act_wtype = a.qtype;
    }
    return true;
}

// The decode-step attention of nn/decoder.rs:1937-2105 as one launch: the
// query / key rows' RMS_NORM -> MUL(w) -> ROPE (node t and the key rows' norm
// after it), the K and V SET_ROWS into the caches and the FLASH_ATTN_EXT over
// them, when nothing else reads the intermediate results and no other node
// runs in between. Falls back (false, nothing planned) on any other shape.
bool planner::plan_attn_step(int i, const ggml_tensor * t) {
    norm_rope_job j0, j1;
    const ggml_tensor *mul0, *rope0, *mul1 = nullptr, *rope1 = nullptr;
    if (!norm_rope_match(i, t, j0, mul0, rope0)) return false;
    const ggml_tensor * t1 = nullptr;
    int i1 = -1;
    for (int j = i + 1; j < cg->n_nodes; j++) {
        const ggml_tensor * n = cg->nodes[j];
        if (is_view_op(n->op) || bypass.count(n) || deferred.count(n) || gqa_skip.count(n) || n == mul0 || n == rope0)
            continue;
        t1 = n;
        i1 = j;
        break;
    }
    if (!t1 || !norm_rope_match(i1, t1, j1, mul1, rope1)) return false;
    if (j0.theta_scale != j1.theta_scale || j0.freq_scale != j1.freq_scale || j0.attn_factor != j1.attn_factor ||
        j0.pos != j1.pos)
        return false;
    // the attention reading the query rows
    const ggml_tensor * F = nullptr;
    int iF = -1;
    for (int j = i1 + 1; j < cg->n_nodes; j++) {
        const ggml_tensor * n = cg->nodes[j];
        if (n->op == GGML_OP_FLASH_ATTN_EXT && root_of(n->src[0]) == rope0) {
            F = n;
            iF = j;
            break;
        }
    }
    if (!F || !supports_op(be->dev, F)) return false;
    // the cache write an attention operand reads: the SET_ROWS itself, or
    // through a GQA expansion that is not launched (its source a reshape of
    // the SET_ROWS with the write's own layout)
    auto set_rows_of = [&](const ggml_tensor * x) -> const ggml_tensor * {
        if (x->op == GGML_OP_SET_ROWS) return x;
        tview v;
        if (!gqa_fold(x, v)) return nullptr;
        const ggml_tensor * src = (x->view_src ? x->view_src : x)->src[0];
        if (src->op != GGML_OP_RESHAPE && src->op != GGML_OP_VIEW) return nullptr;
        const ggml_tensor * sr = src->src[0];
        if (!sr || sr->op != GGML_OP_SET_ROWS || sr->data != v.data || sr->ne[3] != 1 || v.ne[1] != sr->ne[1] ||
            v.ne[2] != sr->ne[2] || v.nb[1] != (int64_t) sr->nb[1] || v.nb[2] != (int64_t) sr->nb[2])
            return nullptr;
        return sr;
    };
    const ggml_tensor *sk = set_rows_of(F->src[1]), *sv = set_rows_of(F->src[2]);
    if (!sk || !sv) return false;
    if (sk->op != GGML_OP_SET_ROWS || sv->op != GGML_OP_SET_ROWS || sk->src[1] != sv->src[1]) return false;
    if (sk->type != GGML_TYPE_F16 || sv->type != GGML_TYPE_F16 || root_of(sk->src[0]) != rope1) return false;
    const ggml_tensor *qv = F->src[0], *kn = sk->src[0], *vn = sv->src[0], *idx = sk->src[1];
    // rope outputs [128, heads, n_seq]; the attention / set_rows views
    // [128, 1, heads, n_seq] over them
    auto head_view = [](const ggml_tensor * v, const ggml_tensor * r) {
        return v->data == r->data && r->ne[3] == 1 && v->ne[0] == 128 && v->ne[1] == 1 && v->ne[2] == r->ne[1] &&
               v->ne[3] == r->ne[2] && v->nb[0] == 4 && v->nb[2] == r->nb[1] && v->nb[3] == r->nb[2];
    };
    if (!head_view(qv, rope0) || !head_view(kn, rope1)) return false;
    if (vn->type != GGML_TYPE_F32 || vn->ne[0] != 128 || vn->ne[1] != 1 || vn->ne[2] != kn->ne[2] ||
        vn->ne[3] != kn->ne[3])
        return false;
    if (sk->ne[2] != kn->ne[2] || sk->ne[3] != kn->ne[3] || sv->ne[2] != vn->ne[2] || sv->ne[3] != vn->ne[3])
        return false;
    if (idx->ne[0] < 1 || idx->ne[3] != 1) return false;
    if (j0.a.ne[3] != 1 || j1.a.ne[3] != 1 || j0.a.nb[0] != 4 || j1.a.nb[0] != 4) return false;
    fattn_args fa;
    if (!make_fattn(F, fa)) return false;
    if (!attn_step_supported(fa)) return false;
    // nothing else runs between the first norm and the attention, and nothing
    // outside the fused nodes reads their intermediate results
    const ggml_tensor * fused[] = {t, mul0, rope0, t1, mul1, rope1, sk, sv, F};
    auto in_fused = [&](const ggml_tensor * n) {
        for (const ggml_tensor * f : fused)
            if (n == f) return true;
        return false;
    };
    for (int j = i + 1; j <= iF; j++) {
        const ggml_tensor * n = cg->nodes[j];
        if (is_view_op(n->op) || bypass.count(n) || in_fused(n) || gqa_skip.count(n)) continue;
        return false;
    }
    for (int j = i + 1; j < cg->n_nodes; j++) {
        const ggml_tensor * n = cg->nodes[j];
        if (is_view_op(n->op) || in_fused(n) || gqa_skip.count(n)) continue;
        for (int k = 0; k < GGML_MAX_SRC; k++) {
            const ggml_tensor * x = n->src[k];
            if (!x) continue;
            for (const ggml_tensor * f : fused) {
                if (f == F) continue;
                if (x == f || (root_of(x) == f && f != sk && f != sv)) return false;
            }
        }
    }
    for (const ggml_tensor * f : fused) {
        if (f != F && (f->flags & GGML_TENSOR_FLAG_OUTPUT)) return false;
    }
    const tview vsrc = view_of(vn);
    attn_step_args as{};
    const ggml_tensor * oview = nullptr;
    fattn_quant_out(iF, F, fa, oview);
    // When the output projection consumes the quantized output this launch
    // writes, nothing reads the f32 output: it goes to scratch, not to F's
    // bytes (which an allocator may well have placed over the projection
    // rows this launch reads). Any other reader of F then fails the plan.
    const bool f32_unread = fa.qtype >= 0 && !(F->flags & GGML_TENSOR_FLAG_OUTPUT) && !no_divert.count(F);
    if (!f32_unread) {
        // the kernel's output must not overlap what it reads (the projection rows)
        uintptr_t lo, hi, olo = (uintptr_t) F->data, ohi = olo + ggml_nbytes(F);
        const tview * reads[] = {&j0.a, &j1.a, &vsrc};
        for (const tview * v : reads) {
            view_span(*v, 4, lo, hi);
            if (lo < ohi && olo < hi) return false;
        }
    }
    as.fa = fa;
    as.qsrc = j0.a.data;
    as.q_nb1 = j0.a.nb[1];
    as.q_nb2 = j0.a.nb[2];
    as.ksrc = j1.a.data;
    as.k_nb1 = j1.a.nb[1];
    as.k_nb2 = j1.a.nb[2];
    as.vsrc = vsrc.data;
    as.v_nb1 = vsrc.nb[2];
    as.v_nb2 = vsrc.nb[3];
    as.qw = j0.w;
    as.kw = j1.w;
    as.q_eps = j0.eps;
    as.k_eps = j1.eps;
    as.pos = j0.pos;
    as.theta_scale = j0.theta_scale;
    as.freq_scale = j0.freq_scale;
    as.attn_factor = j0.attn_factor;
    as.idx = (const char *) idx->data;
    as.idx_nb1 = idx->nb[1];
    as.idx_nb2 = idx->nb[2];
    as.idx_ne1 = (int) idx->ne[1];
    as.idx_ne2 = (int) idx->ne[2];
    as.idx_i64 = idx->type == GGML_TYPE_I64;
    as.kc = (char *) sk->data;
    as.kc_nb1 = sk->nb[1];
    as.kc_nb2 = sk->nb[2];
    as.kc_nb3 = sk->nb[3];
    as.kc_rows = sk->ne[1];
    as.vc = (char *) sv->data;
    as.vc_nb1 = sv->nb[1];
    as.vc_nb2 = sv->nb[2];
    as.vc_nb3 = sv->nb[3];
    as.vc_rows = sv->ne[1];
    as.out = f32_unread ? nullptr : (float *) F->data;  // (nullptr: scratch, set at launch)
    if (fa.n_seq * 64 * sizeof(float2) > kRopeTableBytes) return false;
    for (const ggml_tensor * f : fused) {
        if (f != t) deferred[f] = f;
    }
    const size_t out_off = align_up(attn_step_scratch_bytes(fa), kAlign);
    gen_need = std::max(gen_need, out_off + (f32_unread ? (size_t) ggml_nbytes(F) : 0));
    if (f32_unread) unwritten.insert(F);
    backend_state * b = be;
    // the rotation table of this step's positions, once per graph (again if
    // another layer rotates differently)
    const int64_t qK = (int64_t) fa.d * fa.hq, qN = (int64_t) fa.n_q * fa.n_seq;
    const int n_seq = fa.n_seq;
    if (rope_cur.pos != j0.pos || rope_cur.n_seq != n_seq || rope_cur.theta_scale != j0.theta_scale ||
        rope_cur.freq_scale != j0.freq_scale || rope_cur.attn_factor != j0.attn_factor) {
        rope_cur.pos = j0.pos;
        rope_cur.n_seq = n_seq;
        rope_cur.theta_scale = j0.theta_scale;
        rope_cur.freq_scale = j0.freq_scale;
        rope_cur.attn_factor = j0.attn_factor;
        const rope_key rk = rope_cur;
        add_step([=](hipStream_t s) {
            launch_rope_table((float2 *) rope_base(b), rk.pos, rk.n_seq, rk.theta_scale, rk.freq_scale, rk.attn_factor, s);
        }, F, "rope_table", {nullptr});
    }
    add_step(
        [=](hipStream_t s) {
            attn_step_args la = as;
            la.rope = (const float2 *) rope_base(b);
            if (la.fa.qtype >= 0) la.fa.act = act_carve(la.fa.qtype, act_base(b), qK, qN);
            if (!la.out) la.out = (float *) (gen_base(b) + out_off);
            launch_attn_step(la, gen_base(b), s);
        },
        F, fa.dec ? "attn_step_dec" : "attn_step",
        f32_unread ? std::vector<const ggml_tensor *>{sk, sv} : std::vector<const ggml_tensor *>{F, sk, sv});
    if (fa.qtype >= 0) {
        act_src = oview;
        act_wtype = fa.qtype;
    }
    return true;
}

// One launch for a fused attention chain (find_naive), at its output CONT.
// If the output's bytes overlap what the launch reads (an allocator may
// place it over the query rows, which are dead after the scores product),
// the launch writes to scratch and a copy moves the rows.
bool planner::plan_naive(int i, const ggml_tensor * t) {
    (void) i;
    const naive_job & j = naive_jobs.at(t);
    const naive_attn_args a = j.a;
    const span o = span_of(t);
    bool clash = false;
    for (const auto & r : j.reads) clash = clash || overlap(o, r.first);
    const size_t work = attn_naive_scratch_bytes(a);
    const size_t out_off = align_up(work, kAlign);
    gen_need = std::max(gen_need, out_off + (clash ? (size_t) ggml_nbytes(t) : 0));
    const tview dv = make_view(t);
    backend_state * b = be;
    const int ncu = n_cu;
    add_step(
        [=](hipStream_t s) {
            naive_attn_args la = a;
            char * g = gen_base(b);
            if (clash) la.out = (float *) (g + out_off);
            launch_attn_naive(la, (float *) g, s);
            if (clash) {
                tview sv = dv;
                sv.data = g + out_off;
                launch_copy(dv, GGML_TYPE_F32, sv, GGML_TYPE_F32, s, ncu);
            }
        },
        t, "attn_naive");
    return true;
}

// The plan moves reads later than the graph has them in two places: a
// bypassed CONT's readers read its source at their own positions, and a
// deferred unary node reads its source at its consumer's position. Under an
// allocator that reuses dead blocks, a launch between may already have
// written those bytes. Such a fusion is recorded in no_bypass / no_defer and
// validate returns false, and the caller plans again without it.
bool planner::validate() {
    bool ok = true;
    auto written_between = [&](span src, int from, int to, bool allow_exact_at_to) {
        for (const step & st : steps) {
            if (st.pos <= from || st.pos > to) continue;
            for (const auto & w : st.writes) {
                const span ws{w.first, w.second};
                if (!overlap(ws, src)) continue;
                if (allow_exact_at_to && st.pos == to && ws.lo == src.lo && ws.hi == src.hi) continue;
                return true;
            }
        }
        return false;
    };
    for (const auto & bp : bypass) {
        const ggml_tensor * c = bp.first;
        const tview sv = make_view(bp.second);
        if (written_between(span_of(sv, 4), index.at(c), bypass_last.at(c), false)) {
            no_bypass.insert(c);
            ok = false;
        }
    }
    for (const auto & du : deferred_unary) {
        if (written_between(span_of(du.first->src[0]), index.at(du.first), du.second, true)) {
            no_defer.insert(du.first);
            ok = false;
        }
    }
    // an expansion not launched: its readers read the source later than the
    // REPEAT would have
    for (const fold_read & fr : fold_reads) {
        if (written_between(fr.src, fr.from, fr.to - 1, false)) {
            no_fold.insert(fr.rep);
            ok = false;
        }
    }
    // a fused attention chain reads its operands at its output's position
    for (const auto & nj : naive_jobs) {
        const int at = index.at(nj.first);
        for (const auto & r : nj.second.reads) {
            if (written_between(r.first, r.second, at - 1, false)) {
                no_naive.insert(nj.first);
                ok = false;
                break;
            }
        }
    }
    return ok;
}

bool planner::plan() {
    count_uses();
    find_bypass();
    find_naive();
    find_gqa_skip();
    if (naive_dropped) {
        // a chain dropped after the expansions were decided: decide again without it
        replan = true;
        error = "an attention chain's K and V expansions fold differently";
        return false;
    }
    for (int i = 0; i < cg->n_nodes; i++) {
        const ggml_tensor * t = cg->nodes[i];
        cur = i;
        if (is_view_op(t->op)) continue;
        if (!supports_op(be->dev, t)) return fail(t, "unsupported op or layout");
        if (t->op != GGML_OP_MUL_MAT && !deferred.count(t)) {
            for (int k = 0; k < GGML_MAX_SRC; k++)
                if (t->src[k] && reads_unwritten(t, t->src[k])) return false;
        }
        if (gqa_skip.count(t) || naive_nodes.count(t)) continue;  // read through its source / part of a fused chain
        // a read of an expansion that is not launched must fold into the reader
        for (int k = 0; k < GGML_MAX_SRC; k++) {
            const ggml_tensor * x = t->src[k];
            if (!x || !gqa_skip.count(root_of(x))) continue;
            tview v;
            if (t->op == GGML_OP_FLASH_ATTN_EXT && (k == 1 || k == 2) && gqa_fold(x, v)) continue;
            no_fold.insert(root_of(x));
            replan = true;
            return fail(t, "reads a GQA expansion that is not launched");
        }
        if (bypass.count(t)) continue;  // readers take the CONT's source directly
        auto dit = deferred.find(t);
        if (dit != deferred.end() && dit->second == t) continue;  // produced by a fused predecessor
        if (dit != deferred.end()) continue;                        // evaluated inside its consumer
        const int ncu = n_cu;
        switch (t->op) {
            case GGML_OP_MUL_MAT:
                if (!plan_mul_mat(i, t)) return false;
                continue;
            case GGML_OP_RMS_NORM:
            case GGML_OP_NORM:
                plan_norm(i, t);
                break;
            case GGML_OP_UNARY:
                plan_unary(i, t);
                break;
            case GGML_OP_SIN:
            case GGML_OP_COS: {
                const tview dv = make_view(t), av = make_view(t->src[0]);
                const int code = t->op == GGML_OP_SIN ? kUnarySin : kUnaryCos;
                add_step([=](hipStream_t s) { launch_unary(dv, av, code, nullptr, s, ncu); }, t,
                         t->op == GGML_OP_SIN ? "sin" : "cos");
                break;
            }
            case GGML_OP_CONCAT: {
                const tview dv = make_view(t), av = view_of(t->src[0]), bv = view_of(t->src[1]);
                const int dim = t->op_params[0], es = t->type == GGML_TYPE_F16 ? 2 : 4;
                add_step([=](hipStream_t s) { launch_concat(dv, av, bv, dim, es, s, ncu); }, t, "concat");
                break;
            }
            case GGML_OP_ADD:
            case GGML_OP_SUB:
            case GGML_OP_MUL:
            case GGML_OP_DIV:
                plan_binary(t);
                break;
            case GGML_OP_SCALE: {
                const tview dv = make_view(t), av = make_view(t->src[0]);
                const float sc = op_f32(t, 0), bias = op_f32(t, 1);
                add_step([=](hipStream_t s) { launch_scale(dv, av, sc, bias, s, ncu); }, t, "scale");
                break;
            }
            case GGML_OP_ROPE: {
                const tview dv = make_view(t), av = view_of(t->src[0]);
                const int32_t * pos = (const int32_t *) t->src[1]->data;
                const int n_dims = t->op_params[1], mode = t->op_params[2];
                const float fb = op_f32(t, 5), fs = op_f32(t, 6), af = op_f32(t, 8);
                add_step([=](hipStream_t s) { launch_rope(dv, av, pos, n_dims, mode, fb, fs, af, s, ncu); }, t, "rope");
                break;
            }
            case GGML_OP_SET_ROWS: {
                const tview dv = make_view(t), sv = view_of(t->src[0]), iv = make_view(t->src[1]);
                const int dtype = t->type, i64 = t->src[1]->type == GGML_TYPE_I64;
                // the next planned node writing rows with the same indices
                // (the V write after the K write) shares the launch
                const ggml_tensor * t2 = nullptr;
                for (int j = i + 1; j < cg->n_nodes; j++) {
                    const ggml_tensor * n = cg->nodes[j];
                    if (is_view_op(n->op) || bypass.count(n)) continue;
                    if (n->op == GGML_OP_SET_ROWS && n->src[1] == t->src[1] && supports_op(be->dev, n) &&
                        root_of(n->src[0]) != root_of(t) && n->src[0] != t) {
                        t2 = n;
                    }
                    break;
                }
                if (t2) {
                    const tview dv2 = make_view(t2), sv2 = view_of(t2->src[0]);
                    const int dtype2 = t2->type;
                    deferred[t2] = t2;
                    add_step([=](hipStream_t s) { launch_set_rows(dv, dtype, sv, iv, i64, s, ncu, &dv2, dtype2, &sv2); },
                             t2, "set_rows", {t, t2});
                } else {
                    add_step([=](hipStream_t s) { launch_set_rows(dv, dtype, sv, iv, i64, s, ncu); }, t, "set_rows");
                }
                break;
            }
            case GGML_OP_GET_ROWS: {
                const tview dv = make_view(t), sv = make_view(t->src[0]), iv = make_view(t->src[1]);
                const int stype = t->src[0]->type;
                add_step([=](hipStream_t s) { launch_get_rows(dv, sv, stype, iv, s, ncu); }, t, "get_rows");
                break;
            }
            case GGML_OP_REPEAT: {
                const tview dv = make_view(t), sv = view_of(t->src[0]);
                const int es = (int) ggml_type_size(t->type);
                add_step([=](hipStream_t s) { launch_repeat(dv, sv, es, s, ncu); }, t, "repeat");
                break;
            }
            case GGML_OP_CPY:
            case GGML_OP_CONT:
            case GGML_OP_DUP: {
                if (naive_jobs.count(t)) {
                    if (!plan_naive(i, t)) return false;
                    continue;
                }
                const ggml_tensor * dst = t;
                const tview dv = make_view(dst), av = view_of(t->src[0]);
                const int dtype = dst->type, atype = t->src[0]->type;
                add_step([=](hipStream_t s) { launch_copy(dv, dtype, av, atype, s, ncu); }, t, "copy");
                break;
            }
            case GGML_OP_SOFT_MAX: {
                const tview dv = make_view(t), av = make_view(t->src[0]);
                const bool hm = t->src[1] != nullptr;
                const tview mv = hm ? make_view(t->src[1]) : tview{};
                const float sc = op_f32(t, 0);
                add_step([=](hipStream_t s) { launch_soft_max(dv, av, hm ? &mv : nullptr, sc, s); }, t, "soft_max");
                break;
            }
            case GGML_OP_ARGMAX:
            case GGML_OP_ARGMAX_FIRST: {
                const tview av = make_view(t->src[0]);
                int32_t * out = (int32_t *) t->data;
                const int first = t->op == GGML_OP_ARGMAX_FIRST;
                gen_need = std::max(gen_need, argmax_scratch_bytes(av.ne[0], av.ne[1]));
                backend_state * b = be;
                add_step(
[=](hipStream_t s) {
                        launch_argmax(av, out, first, gen_base(b), s);
                    },
                    t, "argmax");
                break;
            }
            case GGML_OP_IM2COL: {
                const ggml_tensor * kr = t->src[0];
                const tview bv = make_view(t->src[1]);
                const bool two_d = t->op_params[6] != 0;
                im2col_args a{};
                a.total = t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3];
                a.K = t->ne[0], a.OW = t->ne[1];
                a.KW = (int) kr->ne[0], a.KH = two_d ? (int) kr->ne[1] : 1;
                a.s0 = t->op_params[0], a.s1 = t->op_params[1], a.p0 = t->op_params[2], a.p1 = t->op_params[3];
                a.d0 = t->op_params[4], a.d1 = t->op_params[5];
                a.IW = bv.ne[0];
                if (two_d) {
                    a.OH = t->ne[2], a.IH = bv.ne[1], a.nb_h = bv.nb[1], a.nb_c = bv.nb[2], a.nb_n = bv.nb[3];
                } else {
                    a.OH = 1, a.IH = 1, a.nb_h = 0, a.nb_c = bv.nb[1], a.nb_n = bv.nb[2];
                }
                void * d = t->data;
                const int f16 = t->type == GGML_TYPE_F16;
                const char * src = bv.data;
                // read only (through its RESHAPE) as src0 of an F32 x F32
                // column GEMM at the default precision that runs in the
                // aligned bf16 form: written as that form's hi / lo operand
                const ggml_tensor * rs = sole_consumer(t, i + 1);
                const ggml_tensor * mm = rs && rs->op == GGML_OP_RESHAPE && rs->view_src == t ? sole_consumer(rs, i + 1)
                                                                                               : nullptr;
                if (!f16 && t->ne[0] % 8 == 0 && (uintptr_t) d % 16 == 0 && mm && mm->op == GGML_OP_MUL_MAT &&
                    mm->src[0] == rs && mm->src[1] != rs && mm->op_params[0] != GGML_PREC_F32 &&
                    mm->src[1]->type == GGML_TYPE_F32 && mm->type == GGML_TYPE_F32 && supports_op(be->dev, mm)) {
                    const tview rv = make_view(rs), xv2 = make_view(mm->src[1]), mv = make_view(mm);
                    if (gemm_float_supported(mv, rv, GGML_TYPE_F32, xv2, GGML_TYPE_F32) &&
                        gemm_float_x3_aligned(rv, xv2)) {
                        a.split = 1;
                        split_cols.insert(t);
                    }
                }
                add_step([=](hipStream_t s) { launch_im2col(d, f16, src, a, s); }, t, "im2col");
                break;
            }
            case GGML_OP_FLASH_ATTN_EXT:
                if (!plan_fattn(i, t)) return false;
                continue;
            default:
                return fail(t, "no launcher");
        }
        // a node other than MUL_MAT may overwrite memory the act region was
        // quantized from only through a view; be conservative for writers
        if (t->op == GGML_OP_SET_ROWS || t->op == GGML_OP_CPY) act_src = nullptr;
    }
    return true;
}

// plan cg, and plan again without the fusions validate() finds unsafe under
// the graph's allocation (each pass removes at least one; they are few)
std::unique_ptr<planner> make_plan(backend_state * be, const ggml_cgraph * cg, bool & ok) {
    plan_exclusions x;
    for (int pass = 0; pass < 64; pass++) {
        auto p = std::make_unique<planner>(be, cg, x);
        ok = p->plan();
        if (!ok && !p->replan) return p;
        if (ok && p->validate()) return p;
        x = p->exclusions();
    }
    auto p = std::make_unique<planner>(be, cg, x);
    ok = p->plan() && p->validate();
    if (!ok && p->error.empty()) p->error = "no safe plan for this allocation";
    return p;
}

// the arena: two equal halves (activation region, general region), at least
// 32 MiB each
size_t arena_half(size_t act_need, size_t gen_need) {
    act_need = align_up(act_need, kAlign);
    gen_need = align_up(gen_need + kRopeTableBytes, kAlign);
    return std::max<size_t>(std::max(act_need, gen_need), 32u << 20);
}

bool ensure_scratch(backend_state * be, size_t act_need, size_t gen_need) {
    const size_t half = arena_half(act_need, gen_need);
    if (be->scratch && half <= be->gen_off) return true;
    release_scratch(be);
    if (hipMalloc((void **) &be->scratch, 2 * half) != hipSuccess) {
        (void) hipGetLastError();
        be->scratch = nullptr;
        ledger_failure(be->dev);
        return false;
    }
    be->scratch_cap = 2 * half;
    be->gen_off = half;
    ledger_add(be->dev, be->scratch_cap, true);
    return true;
}

enum ggml_status map_error(hipError_t e) {
    if (e == hipSuccess) return GGML_STATUS_SUCCESS;
    if (e == hipErrorLaunchFailure || e == hipErrorIllegalAddress || e == hipErrorECCNotCorrectable ||
        e == hipErrorNoDevice)
        return GGML_STATUS_DEVICE_LOST;
    return GGML_STATUS_EXECUTION_FAILED;
}

}  // namespace

void ledger_add(device_state * dev, uint64_t bytes, bool workspace) {
    std::lock_guard<std::mutex> lk(dev->mem_mu);
    (workspace ? dev->workspace_bytes : dev->live_bytes) += bytes;
    dev->high_water = std::max(dev->high_water, dev->live_bytes + dev->workspace_bytes);
    dev->alloc_count++;
    dev->generation++;
}

void ledger_sub(device_state * dev, uint64_t bytes, bool workspace) {
    std::lock_guard<std::mutex> lk(dev->mem_mu);
    uint64_t & v = workspace ? dev->workspace_bytes : dev->live_bytes;
    v -= std::min(v, bytes);
    dev->generation++;
}

void ledger_failure(device_state * dev) {
    std::lock_guard<std::mutex> lk(dev->mem_mu);
    dev->alloc_failures++;
}

void release_scratch(backend_state * be) {
    release_graph_cache(be);
    if (be->scratch) {
        MI_CHECK(hipFree(be->scratch));
        ledger_sub(be->dev, be->scratch_cap, true);
    }
    be->scratch = nullptr;
    be->scratch_cap = 0;
    be->gen_off = 0;
}

bool graph_arena_bytes(backend_state * be, ggml_cgraph * cg, size_t * bytes) {
    bool ok;
    auto p = make_plan(be, cg, ok);
    if (!ok) return false;
    *bytes = 2 * arena_half(p->act_need, p->gen_need);
    return true;
}

bool reserve_graph_arena(backend_state * be, ggml_cgraph * cg) {
    MI_CHECK(hipSetDevice(be->dev->hip_id));
    bool ok;
    auto p = make_plan(be, cg, ok);
    return ok && ensure_scratch(be, p->act_need, p->gen_need);
}

void release_graph_cache(backend_state * be) {
    for (cache_entry & c : be->cache) {
        if (c.exec) (void) hipGraphExecDestroy(c.exec);
        if (c.graph) (void) hipGraphDestroy(c.graph);
    }
    be->cache.clear();
}

static cache_entry * find_entry(backend_state * be, uint64_t key) {
    for (cache_entry & c : be->cache) {
        if (c.key == key) return &c;
    }
    return nullptr;
}

static cache_entry * new_entry(backend_state * be, uint64_t key) {
    const size_t kMax = 16;
    if (be->cache.size() >= kMax) {
        size_t victim = 0;
        for (size_t i = 1; i < be->cache.size(); i++) {
            if (be->cache[i].last_use < be->cache[victim].last_use) victim = i;
        }
        cache_entry & v = be->cache[victim];
        if (v.exec) (void) hipGraphExecDestroy(v.exec);
        if (v.graph) (void) hipGraphDestroy(v.graph);
        be->cache.erase(be->cache.begin() + (long) victim);
    }
    cache_entry e;
    e.key = key;
    be->cache.push_back(e);
    return &be->cache.back();
}

// the status of a compute that failed with HIP error e; a device-fatal one
// poisons the backend (the host then leaks and never reuses it,
// cpu_graph.rs:7880-7924)
static enum ggml_status fail_with(backend_state * be, hipError_t e, const char * what) {
    std::fprintf(stderr, "mi355x: %s: %s\n", what, hipGetErrorString(e));
    be->last_native_error = (int64_t) e;
    const enum ggml_status st = map_error(e);
    if (st == GGML_STATUS_DEVICE_LOST) be->poisoned = true;
    return st;
}

// run the planned steps on the backend stream; the test seam refuses the
// first one the way a launcher refuses (noted error, nothing enqueued)
static void run_steps(backend_state * be, std::vector<step> & steps, size_t first, size_t last) {
    for (size_t k = first; k < last; k++) {
        if (be->fail_next_launch) {
            be->fail_next_launch = false;
            note_hip_error(hipErrorInvalidValue);
            continue;
        }
        steps[k].run(be->stream);
    }
}

enum ggml_status graph_compute(backend_state * be, ggml_cgraph * cg) {
    if (be->poisoned) return GGML_STATUS_BACKEND_POISONED;
    be->last_native_error = 0;
    // a transfer into this device that failed since the last compute: the
    // graph would read what it failed to write
    const int te = be->dev->transfer_error.exchange(0);
    if (te != 0) return fail_with(be, (hipError_t) te, "an earlier tensor transfer failed");
    be->launch_error.store(0);
    error_scope scope(&be->launch_error);
    MI_CHECK(hipSetDevice(be->dev->hip_id));
    flush_uploads(be->dev, be->stream, false);  // queued input writes land ahead of the graph
    const uint64_t key = graph_key(cg);
    cache_entry * ce = find_entry(be, key);
    be->use_clock++;
    if (ce && ce->exec && !be->abort_cb && !be->fail_next_launch) {
        ce->last_use = be->use_clock;
        be->last_observation = GGML_BACKEND_GRAPH_CANCEL_OBSERVATION_GRAPH_COMPLETION;
        hipError_t e = hipGraphLaunch(ce->exec, be->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(be->stream);
        if (e != hipSuccess) return fail_with(be, e, "graph replay failed");
        return GGML_STATUS_SUCCESS;
    }

    bool planned;
    auto pp = make_plan(be, cg, planned);
    planner & p = *pp;
    if (!planned) {
        std::fprintf(stderr, "mi355x: cannot plan graph: %s\n", p.error.c_str());
        return GGML_STATUS_FAILED;
    }
    if (!ensure_scratch(be, p.act_need, p.gen_need)) return GGML_STATUS_ALLOC_FAILED;
    ce = find_entry(be, key);  // the scratch may have been reallocated, dropping entries
    if (!ce) ce = new_entry(be, key);
    ce->last_use = be->use_clock;
    ce->seen++;

    if (ce->exec) {
        // a cached graph exists but this compute runs the plan (the test seam
        // is armed): the plan is captured afresh below or runs eagerly
        (void) hipGraphExecDestroy(ce->exec);
        (void) hipGraphDestroy(ce->graph);
        ce->exec = nullptr;
        ce->graph = nullptr;
    }
    const bool capture = be->use_graphs && !be->abort_cb && ce->seen >= 2;
    if (capture) {
        hipError_t e = hipStreamBeginCapture(be->stream, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            run_steps(be, p.steps, 0, p.steps.size());
            e = hipStreamEndCapture(be->stream, &ce->graph);
        }
        if (e == hipSuccess && be->launch_error.load() != 0) {
            // a launch was refused while capturing: the graph lacks it and
            // must never be replayed
            (void) hipGraphDestroy(ce->graph);
            ce->graph = nullptr;
            std::fprintf(stderr, "mi355x: a launch was refused: %s\n",
                         hipGetErrorString((hipError_t) be->launch_error.load()));
            be->last_native_error = be->launch_error.load();
            return GGML_STATUS_FAILED;
        }
        if (e == hipSuccess) e = hipGraphInstantiate(&ce->exec, ce->graph, nullptr, nullptr, 0);
        if (e == hipSuccess) {
            be->last_observation = GGML_BACKEND_GRAPH_CANCEL_OBSERVATION_GRAPH_COMPLETION;
            e = hipGraphLaunch(ce->exec, be->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(be->stream);
            if (e != hipSuccess) return fail_with(be, e, "graph launch failed");
            return GGML_STATUS_SUCCESS;
        }
        std::fprintf(stderr, "mi355x: graph capture failed (%s); running eagerly\n", hipGetErrorString(e));
        (void) hipGetLastError();
        if (ce->graph) {
            (void) hipGraphDestroy(ce->graph);
            ce->graph = nullptr;
        }
        ce->exec = nullptr;
        be->use_graphs = false;
        be->launch_error.store(0);
    }

    be->last_observation = GGML_BACKEND_GRAPH_CANCEL_OBSERVATION_SUBMISSION_CHECKPOINT;
    for (size_t k = 0; k < p.steps.size(); k++) {
        if (be->abort_cb && be->abort_cb(be->abort_data)) {
            (void) hipStreamSynchronize(be->stream);
            return GGML_STATUS_ABORTED;
        }
        run_steps(be, p.steps, k, k + 1);
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(be->stream);
    if (e != hipSuccess) return fail_with(be, e, "graph execution failed");
    if (be->launch_error.load() != 0) {
        // the kernels that did launch have finished (synchronized above)
        std::fprintf(stderr, "mi355x: a launch was refused: %s\n",
                     hipGetErrorString((hipError_t) be->launch_error.load()));
        be->last_native_error = be->launch_error.load();
        return GGML_STATUS_FAILED;
    }
    return GGML_STATUS_SUCCESS;
}

enum ggml_status graph_compute_in(backend_state * be, ggml_cgraph * cg, char * scratch, size_t cap) {
    if (be->poisoned) return GGML_STATUS_BACKEND_POISONED;
    be->last_native_error = 0;
    const int te = be->dev->transfer_error.exchange(0);
    if (te != 0) return fail_with(be, (hipError_t) te, "an earlier tensor transfer failed");
    be->launch_error.store(0);
    error_scope scope(&be->launch_error);
    MI_CHECK(hipSetDevice(be->dev->hip_id));
    flush_uploads(be->dev, be->stream, false);  // queued input writes land ahead of the graph
    bool planned;
    auto pp = make_plan(be, cg, planned);
    planner & p = *pp;
    if (!planned) {
        std::fprintf(stderr, "mi355x: cannot plan graph: %s\n", p.error.c_str());
        return GGML_STATUS_FAILED;
    }
    const size_t act = align_up(p.act_need, kAlign), gen = align_up(p.gen_need + kRopeTableBytes, kAlign);
    if (act + gen > cap) {
        std::fprintf(stderr,
                     "mi355x: graph needs %zu bytes of scratch (activations %zu, partials and tables %zu); "
                     "the caller's scratch holds %zu\n",
                     act + gen, act, gen, cap);
        return GGML_STATUS_ALLOC_FAILED;
    }
    struct override_guard {
        backend_state * be;
        ~override_guard() {
            be->scratch_override = nullptr;
            be->override_gen_off = 0;
        }
    } guard{be};
    be->scratch_override = scratch;
    be->override_gen_off = act;
    be->last_observation = GGML_BACKEND_GRAPH_CANCEL_OBSERVATION_SUBMISSION_CHECKPOINT;
    for (size_t k = 0; k < p.steps.size(); k++) {
        if (be->abort_cb && be->abort_cb(be->abort_data)) {
            (void) hipStreamSynchronize(be->stream);
            return GGML_STATUS_ABORTED;
        }
        run_steps(be, p.steps, k, k + 1);
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(be->stream);
    if (e != hipSuccess) return fail_with(be, e, "graph execution failed");
    if (be->launch_error.load() != 0) {
        std::fprintf(stderr, "mi355x: a launch was refused: %s\n",
                     hipGetErrorString((hipError_t) be->launch_error.load()));
        be->last_native_error = be->launch_error.load();
        return GGML_STATUS_FAILED;
    }
    return GGML_STATUS_SUCCESS;
}

int profile_graph(backend_state * be, ggml_cgraph * cg, int iters, float * step_ms, int max_steps, char * labels,
                  int label_cap) {
    MI_CHECK(hipSetDevice(be->dev->hip_id));
    flush_uploads(be->dev, nullptr, true);
    bool planned;
    auto pp = make_plan(be, cg, planned);
    planner & p = *pp;
    if (!planned) {
        std::fprintf(stderr, "mi355x: cannot plan graph: %s\n", p.error.c_str());
        return -1;
    }
    if (!ensure_scratch(be, p.act_need, p.gen_need)) return -1;
    const int n = (int) p.steps.size();
    std::vector<hipEvent_t> ev((size_t) n + 1);
    // timing events without the system-scope fence a default event record
    // adds (it would lengthen every measured interval)
    for (auto & e : ev) MI_CHECK(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    std::vector<double> acc((size_t) n, 0.0);
    // Each iteration first launches a bounded spin kernel (a few ms of GPU
    // wall clock) so that the host has enqueued every launch group and its
    // event before the GPU reaches them: the groups then run back to back as
    // in a graph replay, and an event interval is the group's own run time
    // plus the command processor's dispatch, without host launch gaps.
    const double spin_us = std::min(8000.0, 20.0 * n + 200.0);
    for (int it = 0; it < iters; it++) {
        launch_spin_us(spin_us, be->dev->wall_clock_khz, be->stream);
        MI_CHECK(hipEventRecord(ev[0], be->stream));
        for (int i = 0; i < n; i++) {
            p.steps[(size_t) i].run(be->stream);
            MI_CHECK(hipEventRecord(ev[(size_t) i + 1], be->stream));
        }
        MI_CHECK(hipStreamSynchronize(be->stream));
        for (int i = 0; i < n; i++) {
            float ms = 0.0f;
            MI_CHECK(hipEventElapsedTime(&ms, ev[(size_t) i], ev[(size_t) i + 1]));
            acc[(size_t) i] += ms;
        }
    }
    const bool replayed = false;
    (void) replayed;
    std::fprintf(stderr, "mi355x: profiled %d launch groups x %d iterations (queued behind a spin)\n", n, iters);
    for (auto & e : ev) MI_CHECK(hipEventDestroy(e));
    for (int i = 0; i < n && i < max_steps; i++) {
        if (step_ms) step_ms[i] = (float) (acc[(size_t) i] / (iters > 0 ? iters : 1));
        if (labels && label_cap > 0) {
            std::snprintf(labels + (size_t) i * (size_t) label_cap, (size_t) label_cap, "%s:%s",
                          p.steps[(size_t) i].label.c_str(), p.steps[(size_t) i].node->name);
        }
    }
    return n;
}

// ------------------------------------------------------------ supports_op --

bool supports_op(const device_state * dev, const ggml_tensor * t) {
    (void) dev;
    auto f32 = [](const ggml_tensor * x) { return x && x->type == GGML_TYPE_F32; };
    switch (t->op) {
        case GGML_OP_NONE:
        case GGML_OP_RESHAPE:
        case GGML_OP_VIEW:
        case GGML_OP_PERMUTE:
        case GGML_OP_TRANSPOSE:
            return true;
        case GGML_OP_ADD:
        case GGML_OP_SUB:
        case GGML_OP_MUL:
        case GGML_OP_DIV:
            return f32(t) && f32(t->src[0]) && f32(t->src[1]);
        case GGML_OP_SCALE:
            return f32(t) && f32(t->src[0]);
        case GGML_OP_UNARY: {
            const int u = t->op_params[0];
            const bool op_ok = u == GGML_UNARY_OP_SILU || u == GGML_UNARY_OP_GELU || u == GGML_UNARY_OP_GELU_ERF ||
                               u == GGML_UNARY_OP_RELU || u == GGML_UNARY_OP_TANH || u == GGML_UNARY_OP_SIGMOID ||
                               u == GGML_UNARY_OP_EXP || u == GGML_UNARY_OP_NEG || u == GGML_UNARY_OP_ABS;
            return op_ok && f32(t) && f32(t->src[0]);
        }
        case GGML_OP_SIN:
        case GGML_OP_COS:
            return f32(t) && f32(t->src[0]);
        case GGML_OP_CONCAT: {
            const int ty = t->type, dim = t->op_params[0];
            return (ty == GGML_TYPE_F32 || ty == GGML_TYPE_F16) && t->src[0]->type == ty && t->src[1]->type == ty &&
                   dim >= 0 && dim < 4;
        }
        case GGML_OP_RMS_NORM:
        case GGML_OP_NORM:
            return f32(t) && f32(t->src[0]) && rows_contiguous(t->src[0], 4) && rows_contiguous(t, 4) &&
                   norm_supported(t->ne[0]);
        case GGML_OP_MUL_MAT: {
            const ggml_tensor *w = t->src[0], *x = t->src[1];
            if (!f32(t) || !is_contiguous(t)) return false;
            // f16 columns (an f16 convolution's IM2COL) only on the matrix-core GEMM
            if (x->type == GGML_TYPE_F16)
                return (w->type == GGML_TYPE_F16 || w->type == GGML_TYPE_F32) &&
                       gemm_float_supported(make_view(t), make_view(w), w->type, make_view(x), x->type);
            if (!f32(x)) return false;
            if (w->type == GGML_TYPE_Q8_0 || w->type == GGML_TYPE_Q4_K) {
                return w->ne[2] == 1 && w->ne[3] == 1 && is_contiguous(w) && columns_foldable(x) &&
                       (w->type != GGML_TYPE_Q4_K || w->ne[0] % 256 == 0) && w->ne[0] % 32 == 0;
            }
            if (w->type == GGML_TYPE_Q3_K)
                return w->ne[2] == 1 && w->ne[3] == 1 && is_contiguous(w) && columns_foldable(x) &&
                       w->ne[0] % 256 == 0;
            return w->type == GGML_TYPE_F16 || w->type == GGML_TYPE_F32;
        }
        case GGML_OP_GET_ROWS: {
            const ggml_tensor * s = t->src[0];
            const bool st = s->type == GGML_TYPE_F32 || s->type == GGML_TYPE_F16 || s->type == GGML_TYPE_Q8_0 ||
                            s->type == GGML_TYPE_Q4_K || s->type == GGML_TYPE_I32;
            const bool rows_ok = (s->type != GGML_TYPE_Q8_0 && s->type != GGML_TYPE_Q4_K) ||
                                 (size_t) s->nb[1] == (size_t) (s->type == GGML_TYPE_Q8_0 ? q8_0_row_bytes(s->ne[0])
                                                                                          : (s->ne[0] / 256) * 144);
            return st && rows_ok && t->src[1]->type == GGML_TYPE_I32;
        }
        case GGML_OP_SET_ROWS:
            return (t->type == GGML_TYPE_F16 || t->type == GGML_TYPE_F32) && f32(t->src[0]) &&
                   (t->src[1]->type == GGML_TYPE_I32 || t->src[1]->type == GGML_TYPE_I64);
        case GGML_OP_ROPE: {
            const int mode = t->op_params[2];
            const float ext = op_f32(t, 7);
            return f32(t) && f32(t->src[0]) && t->src[2] == nullptr && ext == 0.0f &&
                   (mode == GGML_ROPE_TYPE_NEOX || mode == GGML_ROPE_TYPE_NORMAL) && t->op_params[1] % 2 == 0 &&
                   t->op_params[1] <= t->ne[0];
        }
        case GGML_OP_FLASH_ATTN_EXT: {
            const ggml_tensor *q = t->src[0], *k = t->src[1], *v = t->src[2], *m = t->src[3];
            // f32 K / V (strided views straight from the projections, as the
            // encoders pass them) are rounded to contiguous f16 first
            auto kv_ok = [](const ggml_tensor * x) {
                return (x->type == GGML_TYPE_F16 && x->nb[0] == 2) || (x->type == GGML_TYPE_F32 && x->nb[0] == 4);
            };
            if (!f32(q) || q->nb[0] != 4 || !kv_ok(k) || !kv_ok(v)) return false;
            if (v->ne[0] != k->ne[0] || k->ne[2] != v->ne[2]) return false;
            if (op_f32(t, 1) != 0.0f || op_f32(t, 2) != 0.0f) return false;  // max_bias, softcap
            if (m && (m->type != GGML_TYPE_F16 || m->ne[2] != 1 || m->nb[0] != 2)) return false;
            if (q->ne[3] % k->ne[3] != 0) return false;
            return fattn_supported((int) q->ne[0], (int) q->ne[2], (int) k->ne[2]) && is_contiguous(t);
        }
        case GGML_OP_SOFT_MAX:
            return f32(t) && f32(t->src[0]) && op_f32(t, 1) == 0.0f &&
                   (t->src[1] == nullptr || t->src[1]->type == GGML_TYPE_F16);
        case GGML_OP_ARGMAX:
        case GGML_OP_ARGMAX_FIRST:
            return f32(t->src[0]) && rows_contiguous(t->src[0], 4) && t->type == GGML_TYPE_I32;
        case GGML_OP_IM2COL: {
            const ggml_tensor *kr = t->src[0], *b = t->src[1];
            if (!kr || !b || !f32(b) || b->nb[0] != 4 || !is_contiguous(t)) return false;
            if (t->type != GGML_TYPE_F16 && t->type != GGML_TYPE_F32) return false;
            const bool two_d = t->op_params[6] != 0;
            const int64_t K = two_d ? kr->ne[0] * kr->ne[1] * kr->ne[2] : kr->ne[0] * kr->ne[1];
            return t->ne[0] == K && (!two_d || b->nb[1] == 4 * b->ne[0]) && t->ne[1] >= 1 &&
                   t->op_params[0] > 0 && t->op_params[4] > 0 && (!two_d || (t->op_params[1] > 0 && t->op_params[5] > 0));
        }
        case GGML_OP_CPY:
        case GGML_OP_CONT:
        case GGML_OP_DUP: {
            const int a = t->src[0]->type, d = t->type;
            auto ok = [](int ty) { return ty == GGML_TYPE_F32 || ty == GGML_TYPE_F16; };
            return (ok(a) && ok(d)) || (a == GGML_TYPE_I32 && d == GGML_TYPE_I32);
        }
        case GGML_OP_REPEAT: {
            // the GQA K/V expansion (nn/decoder.rs:1799-1841) and any other
            // tiling of 2- or 4-byte elements
            const ggml_tensor * a = t->src[0];
            const bool ty = a->type == t->type && (t->type == GGML_TYPE_F32 || t->type == GGML_TYPE_F16 ||
                                                   t->type == GGML_TYPE_I32);
            bool tiles = true;
            for (int d = 0; d < 4; d++) tiles = tiles && a->ne[d] > 0 && t->ne[d] % a->ne[d] == 0;
            return ty && tiles;
        }
        default:
            return false;
    }
}

}  // namespace mi355x
