"""The graph allocator of the ggml-base shim against the rules a lifetime
allocator must keep (the plugin's fused launches are checked against the
aliasing this allocator produces, so it must produce the same kinds of
aliasing ggml-alloc does): a tensor's bytes are shared only by tensors whose
lifetimes do not overlap, except that an in-place-capable op may take over
the block of a source whose last use it is; inputs and outputs are never
reused; and memory is actually reused. Runs on the host buffer type, no GPU.
"""

import ctypes as C

import numpy as np

INPLACE_OPS = {"SCALE", "ADD", "SUB", "MUL", "DIV", "UNARY", "ROPE", "RMS_NORM", "SOFT_MAX"}
VIEW_OPS = {"NONE", "RESHAPE", "VIEW", "PERMUTE", "TRANSPOSE"}


def op_names(lib):
    lib.ggml_op_name.restype = C.c_char_p
    lib.ggml_op_name.argtypes = [C.c_int]
    return lambda code: lib.ggml_op_name(code).decode()


def allocate_on_host(ggml, G):
    lib = G.lib
    buft = lib.ggml_backend_cpu_buffer_type()
    G.galloc = lib.ggml_gallocr_new(buft)
    assert lib.ggml_gallocr_alloc_graph(G.galloc, G.gf)
    return lib.ggml_gallocr_get_buffer_size(G.galloc, 0)


def check_lifetimes(ggml, G, inputs):
    """Every pair of placed tensors whose byte ranges overlap has disjoint
    lifetimes, or is an in-place handover at the source's last use."""
    lib = G.lib
    name = op_names(lib)
    n = lib.ggml_graph_n_nodes(G.gf)
    nodes = [lib.ggml_graph_node(G.gf, i) for i in range(n)]
    galloc_buffer = None
    info = {}  # tensor address -> [def, last, lo, hi, op, srcs]
    for p in inputs:
        t = ggml.tensor(p)
        if not t.data:  # an input no node reads is never placed
            continue
        info[p] = [-1, n, t.data, t.data + lib.ggml_nbytes(p), "INPUT", []]
        galloc_buffer = t.buffer
    for i, p in enumerate(nodes):
        t = ggml.tensor(p)
        if t.view_src or name(t.op) in VIEW_OPS:
            continue
        if t.buffer != galloc_buffer:
            continue
        last = n if t.flags & 2 else i
        info[p] = [i, last, t.data, t.data + lib.ggml_nbytes(p), name(t.op),
                   [s for s in t.src if s]]
    roots = lambda s: ggml.tensor(s).view_src or s  # ggml keeps the root base in view_src
    for i, p in enumerate(nodes):
        t = ggml.tensor(p)
        for s in t.src:
            if s and roots(s) in info:
                info[roots(s)][1] = max(info[roots(s)][1], i)
        if t.view_src and (t.flags & 2) and t.view_src in info:
            info[t.view_src][1] = n
    items = list(info.items())
    shared = inplace = 0
    for a in range(len(items)):
        pa, (da, la, loa, hia, _, _) = items[a]
        for b in range(a + 1, len(items)):
            pb, (db, lb, lob, hib, opb, srcb) = items[b]
            if not (loa < hib and lob < hia):
                continue
            shared += 1
            if la < db or lb < da:
                continue  # one is dead before the other is defined
            # the only allowed overlap of live ranges: b takes over a's block
            # at a's last use, in place
            ok = (db == la and lob == loa and opb in INPLACE_OPS and any(roots(s) == pa for s in srcb))
            ok = ok or (da == lb and loa == lob and items[a][1][4] in INPLACE_OPS and
                        any(roots(s) == pb for s in items[a][1][5]))
            assert ok, f"live tensors share bytes: {items[a][1]} and {items[b][1]}"
            inplace += 1
    return shared, inplace


def test_layer_graph_reuses_and_goes_in_place(ggml):
    """A decoder-layer-shaped graph: the residual ADD runs in place on the
    projection it consumes, dead intermediates hand their blocks on, and
    neither the input nor an output is ever written by a later node."""
    G = ggml.Graph()
    L = G.lib
    d, f, n = 256, 512, 4
    x = G.new(ggml.F32, d, n)
    wq = G.new(ggml.F32, d, d, weight=True)
    wg = G.new(ggml.F32, d, f, weight=True)
    wu = G.new(ggml.F32, d, f, weight=True)
    wd = G.new(ggml.F32, f, d, weight=True)
    h = L.ggml_rms_norm(G.ctx, x, 1e-6)
    a = L.ggml_mul_mat(G.ctx, wq, h)
    y = L.ggml_add(G.ctx, a, x)  # a's only consumer: in place on a
    h2 = L.ggml_rms_norm(G.ctx, y, 1e-6)
    g = L.ggml_silu(G.ctx, L.ggml_mul_mat(G.ctx, wg, h2))
    u = L.ggml_mul_mat(G.ctx, wu, h2)
    m = L.ggml_mul(G.ctx, g, u)
    z = L.ggml_add(G.ctx, L.ggml_mul_mat(G.ctx, wd, m), y)
    G.build(z)
    G.lib.ggml_backend_alloc_ctx_tensors_from_buft(G.wctx, L.ggml_backend_cpu_buffer_type())
    size = allocate_on_host(ggml, G)
    sizes = [d * n * 4] * 5 + [f * n * 4] * 4 + [d * n * 4] * 2  # every tensor its own block
    assert size < sum(sizes)
    assert ggml.tensor(y).data == ggml.tensor(a).data
    shared, inplace = check_lifetimes(ggml, G, [x])
    assert shared > 0 and inplace > 0
    # the input is live for the whole graph and the output is never shared
    xd = ggml.tensor(x).data
    for i in range(L.ggml_graph_n_nodes(G.gf)):
        t = ggml.tensor(L.ggml_graph_node(G.gf, i))
        if not t.view_src:
            assert t.data != xd
    G.free()


def test_outputs_are_not_taken_in_place(ggml):
    G = ggml.Graph()
    L = G.lib
    x = G.new(ggml.F32, 64, 2)
    w = G.new(ggml.F32, 64, 64, weight=True)
    a = L.ggml_mul_mat(G.ctx, w, x)
    b = L.ggml_scale(G.ctx, a, 2.0)
    L.ggml_set_output(a)
    G.build(b, a)
    G.lib.ggml_backend_alloc_ctx_tensors_from_buft(G.wctx, L.ggml_backend_cpu_buffer_type())
    allocate_on_host(ggml, G)
    assert ggml.tensor(b).data != ggml.tensor(a).data
    # an input is never taken in place either
    G2 = ggml.Graph()
    x2 = G2.new(ggml.F32, 64, 2)
    c = G2.lib.ggml_scale(G2.ctx, x2, 3.0)
    G2.build(c)
    allocate_on_host(ggml, G2)
    assert ggml.tensor(c).data != ggml.tensor(x2).data
    G.free()
    G2.free()


def test_random_graphs_keep_lifetimes_apart(ggml):
    """Seeded random DAGs of elementwise, norm, softmax, matmul, copy and view
    nodes (with random outputs): the liveness invariant holds and blocks are
    reused."""
    for seed in range(12):
        rng = np.random.default_rng(seed)
        G = ggml.Graph()
        L = G.lib
        d, n = 32, 3
        inputs = [G.new(ggml.F32, d, n) for _ in range(2)]
        w = G.new(ggml.F32, d, d, weight=True)
        pool = list(inputs)
        made = []
        for _ in range(40):
            k = int(rng.integers(0, 9))
            a = pool[int(rng.integers(0, len(pool)))]
            b = pool[int(rng.integers(0, len(pool)))]
            if k == 0:
                t = L.ggml_add(G.ctx, a, b)
            elif k == 1:
                t = L.ggml_mul(G.ctx, a, b)
            elif k == 2:
                t = L.ggml_silu(G.ctx, a)
            elif k == 3:
                t = L.ggml_scale(G.ctx, a, 0.5)
            elif k == 4:
                t = L.ggml_rms_norm(G.ctx, a, 1e-6)
            elif k == 5:
                t = L.ggml_mul_mat(G.ctx, w, a)
            elif k == 6:
                t = L.ggml_cont(G.ctx, L.ggml_transpose(G.ctx, L.ggml_cont(G.ctx, L.ggml_transpose(G.ctx, a))))
            elif k == 7:
                t = L.ggml_soft_max(G.ctx, a)
            else:
                t = L.ggml_reshape_2d(G.ctx, L.ggml_cont(G.ctx, a), d, n)
            pool.append(t)
            made.append(t)
            if len(pool) > 6:
                pool.pop(int(rng.integers(0, len(pool) - 2)))
        outs = [made[-1]] + [made[int(i)] for i in rng.integers(0, len(made), 2)]
        G.build(*outs)
        G.lib.ggml_backend_alloc_ctx_tensors_from_buft(G.wctx, L.ggml_backend_cpu_buffer_type())
        allocate_on_host(ggml, G)
        shared, _ = check_lifetimes(ggml, G, inputs)
        assert shared > 0, f"seed {seed}: no block was reused"
        G.free()
