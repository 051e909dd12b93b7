"""The physical-memory ABI v1 on the device, driven the way the host's
wrapper drives it (crates/openasr-core/src/ggml_runtime/backend_memory.rs:
140-330): domains, stats, quotes for BUFFER and GRAPH_PRIVATE requests,
reserve_private against a fresh and a stale quote, trim and quarantine.
"""

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MiB = 1 << 20


@pytest.fixture(scope="module")
def mem(ggml, gpu):
    return ggml.MemoryApi(gpu.reg, gpu.dev, gpu.backend)


def stats1(mem):
    s = mem.stats()
    assert len(s) == 1
    return s[0]


def test_one_device_local_domain(ggml, mem):
    print("memory abi domains", flush=True)
    d = mem.domains()
    assert len(d) == 1
    assert d[0].id.kind == ggml.MEM_DOMAIN_DEVICE_LOCAL and d[0].id.heap_index == 0
    assert any(d[0].id.physical_device_uuid)  # the host refuses an all-zero identity
    assert d[0].name.startswith(b"ROCm")


def test_stats_are_consistent_and_stable(ggml, mem):
    print("memory abi stats", flush=True)
    a, b = stats1(mem), stats1(mem)
    assert a.generation == b.generation  # no allocation in between
    assert not (a.flags & ggml.MEM_STATS_BUDGET_UNAVAILABLE)
    assert a.total_bytes > 200 * (1 << 30) and a.budget_bytes == a.total_bytes
    assert a.device_used_bytes + a.device_free_bytes == a.total_bytes
    assert a.health == ggml.MEM_HEALTHY
    # at least the plugin's GELU table and the fixed scratch array of the
    # allocation-free compute, which every device holds until the process ends
    fn = ggml.plugin().cdll.ggml_backend_mi355x_static_scratch_bytes
    fn.restype = C.c_size_t
    static = fn()
    assert static == 64 * MiB
    assert a.backend_owned_live_bytes >= static + 65536 * 2
    assert a.backend_owned_high_water_bytes >= a.backend_owned_live_bytes + a.backend_owned_workspace_bytes
    assert bytes(a.domain.physical_device_uuid) == bytes(mem.domains()[0].id.physical_device_uuid)


def test_buffer_quote_then_allocation(ggml, gpu, mem):
    print("memory abi buffer quote", flush=True)
    lib = ggml.base()
    s0 = stats1(mem)
    req = ggml.mem_request_of(ggml.MEM_REQUEST_BUFFER, buft=gpu.buft, requested=100 * MiB + 3, request_id=7,
                              usage=ggml.BUFFER_USAGE_WEIGHTS)
    q, claims = mem.quote([req])
    assert q.stats_generation == s0.generation and q.quote_token != 0
    assert len(claims) == 1
    c = claims[0]
    assert c.request_id == 7 and c.payload_requested_bytes == 100 * MiB + 3
    assert c.committed_before_bytes == s0.backend_owned_live_bytes + s0.backend_owned_workspace_bytes
    assert c.commit_peak_extra_upper_bytes == 102 * MiB  # rounded up to the 2 MiB granule
    assert c.flags & ggml.MEM_CLAIM_CONSERVATIVE_UPPER
    assert c.resident_after_upper_bytes == c.committed_before_bytes + c.commit_peak_extra_upper_bytes
    # BUFFER requests are engine-owned: nothing to reserve privately
    assert mem.reserve_private([req], q) == []
    buf = lib.ggml_backend_buft_alloc_buffer(gpu.buft, 100 * MiB + 3)
    assert buf
    try:
        s1 = stats1(mem)
        assert s1.generation != s0.generation
        grew = s1.backend_owned_live_bytes - s0.backend_owned_live_bytes
        assert 100 * MiB + 3 <= grew <= c.commit_peak_extra_upper_bytes
        assert s1.allocation_count == s0.allocation_count + 1
    finally:
        lib.ggml_backend_buffer_free(buf)
    assert stats1(mem).backend_owned_live_bytes == s0.backend_owned_live_bytes
    # a host-import request is refused: the device has no buffer_from_host_ptr
    with pytest.raises(ggml.MemoryStatusError):
        mem.quote([ggml.mem_request_of(ggml.MEM_REQUEST_HOST_IMPORT, buft=gpu.buft, requested=MiB)])


def small_graph(ggml, M=1024, K=2048, N=8):
    G = ggml.Graph()
    W = G.new(ggml.Q4_K, K, M, weight=True)
    X = G.new(ggml.F32, K, N)
    Y = G.lib.ggml_mul_mat(G.ctx, W, X)
    G.build(Y)
    return G, W, X, Y


def test_graph_private_quote_reserve_trim(ggml, gpu, mem, ref):
    print("memory abi graph private", flush=True)
    G, W, X, Y = small_graph(ggml)
    G.allocate(gpu.buft)
    rng = np.random.default_rng(3)
    w = ref.quantize_weights(ref.Q4_K, (rng.standard_normal((1024, 2048)) * 0.02).astype(np.float32))
    x = rng.standard_normal((8, 2048)).astype(np.float32)
    G.set(W, w)
    G.set(X, x)
    mem.trim()
    s0 = stats1(mem)
    assert s0.backend_owned_workspace_bytes == 0
    req = ggml.mem_request_of(ggml.MEM_REQUEST_GRAPH_PRIVATE, backend=gpu.backend, graph=G.gf, request_id=11)
    q, claims = mem.quote([req])
    assert len(claims) == 1 and claims[0].flags & ggml.MEM_CLAIM_EXACT
    arena = claims[0].payload_requested_bytes
    assert arena >= 64 * MiB and claims[0].commit_peak_extra_upper_bytes == arena
    assert q.flags & ggml.MEM_QUOTE_OPAQUE_DRIVER_COSTS
    # the sizing call changes nothing; the commit allocates exactly the quote
    n = C.c_uint32(0)
    reqs = (ggml.mem_request * 1)(req)
    assert mem.raw.reserve_private(reqs, 1, C.byref(q), None, C.byref(n)) == 0 and n.value == 1
    assert stats1(mem).generation == s0.generation
    got = mem.reserve_private([req], q)
    assert len(got) == 1 and got[0].payload_requested_bytes == arena
    s1 = stats1(mem)
    assert s1.backend_owned_workspace_bytes == arena
    # the reserved arena is the one the graph runs in: no growth on compute
    assert G.compute(gpu.backend) == 0
    assert stats1(mem).backend_owned_workspace_bytes == arena
    y = G.get(Y)
    want = ref.mul_mat(ref.Q4_K, w, 1024, 2048, x)
    assert np.array_equal(y.reshape(8, 1024).view(np.uint32), want.reshape(8, 1024).view(np.uint32))
    # a quote taken before an allocation is stale afterwards
    q2, claims2 = mem.quote([req])
    assert claims2[0].commit_peak_extra_upper_bytes == 0  # the arena already fits
    buf = ggml.base().ggml_backend_buft_alloc_buffer(gpu.buft, MiB)
    try:
        with pytest.raises(ggml.MemoryStatusError):
            mem.reserve_private([req], q2)
    finally:
        ggml.base().ggml_backend_buffer_free(buf)
    # trim releases the arena; the next compute grows it again
    mem.trim()
    assert stats1(mem).backend_owned_workspace_bytes == 0
    assert G.compute(gpu.backend) == 0
    assert np.array_equal(G.get(Y), y)
    G.free()


def test_quarantine_fails_closed(ggml, gpu):
    print("memory abi quarantine", flush=True)
    lib = ggml.base()
    be = lib.ggml_backend_dev_init(gpu.dev, None)
    assert be
    try:
        m = ggml.MemoryApi(gpu.reg, gpu.dev, be)
        assert m.stats()[0].health == ggml.MEM_HEALTHY
        m.quarantine(reason=1, status=2, message=b"test quarantine")
        s = m.stats()[0]
        assert s.health == ggml.MEM_QUARANTINED and s.quarantine_generation == 1 and s.last_ggml_status == 2
        G, W, X, Y = small_graph(ggml, M=256, K=256, N=1)
        G.allocate(gpu.buft)
        assert G.compute(be) == 4  # GGML_STATUS_BACKEND_POISONED
        G.free()
    finally:
        lib.ggml_backend_free(be)
