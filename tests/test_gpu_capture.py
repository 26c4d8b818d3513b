"""HIP graph capture through the C-ABI (accel_hip_capture_begin/end, accel_hip_graph_launch):
what a capture must refuse, and stale graphs.

* A call that would allocate, free, synchronize or memset while the library stream is being
  captured returns ACCEL_HIP_RUNTIME_ERROR and enqueues nothing: building a staged weight copy
  (the GEMV's first use of W), growing the split-K workspace, Allocate, the counted copies.
  The same call made eagerly afterwards gives the correct product (no half-built copy left
  behind).
* A graph whose capture read a staged weight copy is refused at launch once that copy has
  been dropped (W rewritten or freed): the launch returns ACCEL_HIP_RUNTIME_ERROR and the
  graph is never replayed. A graph that did not read the dropped copy still replays.
* The fp32 GEMM's staged bf16 parts of a weight (built on its second use) give the same bits
  as the split on the fly, and a graph that read them is refused once they are dropped.

* An event recorded during a capture becomes a node of the graph that every replay records,
  and stays timeable (the bench times its steps between two such events).

No test here replays a graph whose memory was released: every refusal is decided on the host
before anything is launched.
"""

import ctypes as C

import numpy as np
import pytest

from hip_helpers import Buffer, HipError, assert_gamma_bound, check, dequant_host, dev, lib, quant_plane, same_bits

pytestmark = pytest.mark.gpu

RUNTIME_ERROR = 5


@pytest.fixture(scope="module", autouse=True)
def device():
    check(lib().accel_hip_init())
    yield


def _gemv(m, k, n, seed):
    r = np.random.default_rng(seed)
    q = r.integers(-127, 128, size=k * n, dtype=np.int8)
    s = r.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    a = r.standard_normal((m, k)).astype(np.float32)
    qd, sd, ad = dev(q), dev(s), dev(a)
    plane = quant_plane(qd, sd, None, [k, n], 1)
    out = dev(np.zeros((m, n), np.float32))
    w = dequant_host(dict(q=q, scale=s, zero=None, shape=[k, n], axis=1, offset=0), k, n)
    return dict(q=q, s=s, a=a, qd=qd, sd=sd, ad=ad, plane=plane, out=out, w=w, m=m, k=k, n=n)


def _call(g):
    return lib().accel_hip_matmul_quantized(g["ad"].ptr, None, None, C.byref(g["plane"]), g["out"].ptr, g["m"],
                                            g["k"], g["n"])


def _end_capture():
    handle = C.c_void_p()
    check(lib().accel_hip_capture_end(C.byref(handle)))
    return handle


@pytest.mark.parametrize("m", [1, 4])
def test_capture_refuses_first_use_staging(m):
    """The first GEMV on a weight builds its staged copy; inside a capture that is refused, and
    an eager call after the capture (before any replay) computes the right product."""
    L = lib()
    g = _gemv(m, 1024, 2048, 10 + m)
    print(f"capture staging m={m}", flush=True)
    check(L.accel_hip_capture_begin())
    try:
        rc = _call(g)
        msg = L.accel_hip_last_error().decode()
    finally:
        graph = _end_capture()
        check(L.accel_hip_graph_destroy(graph))
    assert rc == RUNTIME_ERROR, (rc, msg)
    assert "captur" in msg and "staging" in msg
    check(_call(g))
    assert_gamma_bound(g["out"].numpy(), g["a"], g["w"])


def test_capture_refuses_heap_calls_and_workspace_growth():
    L = lib()
    target = dev(np.zeros(4, np.float32))
    host = np.arange(4, dtype=np.float32)
    check(L.accel_hip_capture_begin())
    try:
        b = Buffer()
        rc_alloc = L.accel_hip_allocate(256, C.byref(b))
        msg_alloc = L.accel_hip_last_error().decode()
        rc_copy = L.accel_hip_copy_h2d(target.buffer, host.ctypes.data, host.nbytes)
        msg_copy = L.accel_hip_last_error().decode()
    finally:
        graph = _end_capture()
        check(L.accel_hip_graph_destroy(graph))
    assert rc_alloc == RUNTIME_ERROR and "Allocate" in msg_alloc, (rc_alloc, msg_alloc)
    assert rc_copy == RUNTIME_ERROR and "CopyHostToDevice" in msg_copy, (rc_copy, msg_copy)
    assert not target.numpy().any()  # the refused copy wrote nothing
    # A split-K GEMM (64 tiles of 64 x 64, K split 8 ways: 8 MB of partial sums). If no earlier
    # call grew the workspace that far, the capture refuses to grow it and enqueues nothing;
    # either way the eager call afterwards gives the product.
    m, k, n = 64, 8192, 4096
    r = np.random.default_rng(3)
    a_h = r.standard_normal((m, k)).astype(np.float32)
    b_h = (r.standard_normal((k, n)) * 0.02).astype(np.float32)
    a, bw, c = dev(a_h), dev(b_h), dev(np.zeros((m, n), np.float32))
    check(L.accel_hip_capture_begin())
    try:
        rc = L.accel_hip_matmul_fused(a.ptr, bw.ptr, c.ptr, m, k, n, None)
        msg = L.accel_hip_last_error().decode()
    finally:
        graph = _end_capture()
        check(L.accel_hip_graph_destroy(graph))
    if rc != 0:
        assert rc == RUNTIME_ERROR and "workspace" in msg, (rc, msg)
    check(L.accel_hip_matmul_fused(a.ptr, bw.ptr, c.ptr, m, k, n, None))
    assert_gamma_bound(c.numpy(), a_h, b_h)


@pytest.mark.parametrize("m", [1, 4])
def test_graph_refused_after_its_staged_copy_is_dropped(m):
    """Capture a GEMV that reads W's staged copy; rewrite W (which drops the copy): the launch
    of the old graph is refused and nothing runs. A second graph over another weight, whose
    copy was not dropped, still replays with the eager bits. Re-capturing after the rewrite
    gives the new product."""
    L = lib()
    g1 = _gemv(m, 512, 1536, 30 + m)
    g2 = _gemv(m, 512, 1536, 40 + m)
    for g in (g1, g2):
        check(_call(g))  # stages W before the capture
    want2 = g2["out"].numpy()
    check(L.accel_hip_capture_begin())
    try:
        check(_call(g1))
    finally:
        graph1 = _end_capture()
    check(L.accel_hip_capture_begin())
    try:
        check(_call(g2))
    finally:
        graph2 = _end_capture()
    try:
        check(L.accel_hip_graph_launch(graph1, 1))  # still current
        assert_gamma_bound(g1["out"].numpy(), g1["a"], g1["w"])
        q_new = np.random.default_rng(99).integers(-127, 128, size=g1["k"] * g1["n"], dtype=np.int8)
        g1["qd"].upload(q_new)  # drops the staged copy graph1 reads
        g1["out"].upload(np.full((m, g1["n"]), 7.0, np.float32))
        print(f"launching stale graph m={m} (must be refused on the host)", flush=True)
        rc = L.accel_hip_graph_launch(graph1, 1)
        msg = L.accel_hip_last_error().decode()
        assert rc == RUNTIME_ERROR and "stale" in msg, (rc, msg)
        assert (g1["out"].numpy() == 7.0).all()  # nothing ran
        g2["out"].upload(np.zeros((m, g2["n"]), np.float32))
        check(L.accel_hip_graph_launch(graph2, 2))  # its copy is alive
        same_bits(g2["out"].numpy(), want2)
        check(L.accel_hip_graph_destroy(graph1))
        graph1 = None
        check(_call(g1))  # restages
        w_new = dequant_host(dict(q=q_new, scale=g1["s"], zero=None, shape=[g1["k"], g1["n"]], axis=1, offset=0),
                             g1["k"], g1["n"])
        want1 = g1["out"].numpy()
        assert_gamma_bound(want1, g1["a"], w_new)
        check(L.accel_hip_capture_begin())
        try:
            check(_call(g1))
        finally:
            graph1 = _end_capture()
        g1["out"].upload(np.zeros((m, g1["n"]), np.float32))
        check(L.accel_hip_graph_launch(graph1, 1))
        same_bits(g1["out"].numpy(), want1)
    finally:
        if graph1 is not None:
            check(L.accel_hip_graph_destroy(graph1))
        check(L.accel_hip_graph_destroy(graph2))


def test_capture_inside_capture_is_refused():
    L = lib()
    check(L.accel_hip_capture_begin())
    try:
        rc = L.accel_hip_capture_begin()
        msg = L.accel_hip_last_error().decode()
    finally:
        graph = _end_capture()
        check(L.accel_hip_graph_destroy(graph))
    assert rc == RUNTIME_ERROR and "already" in msg
    with pytest.raises(HipError):
        check(L.accel_hip_graph_launch(None, 1))


INVALID_ARGUMENT = 1
STAGE_TILES, STAGE_GROUPS, STAGE_BF16, STAGE_SMALL = 1, 2, 4, 8


def _prepare(plane, k, n, layouts=0):
    staged = C.c_uint32(0xFFFF)
    rc = lib().accel_hip_prepare_quantized(C.byref(plane), k, n, layouts, C.byref(staged))
    return rc, staged.value


def test_prepared_weight_can_be_captured():
    """accel_hip_prepare_quantized builds a weight's staged copies before any use. A capture
    of GEMVs on it (m = 1 on the 8-column tiles, m = 4 on the group-interleaved copy) then
    records, and three replays, each after eager work of its own, store the eager call's
    bits."""
    L = lib()
    k, n = 576, 1536
    g1 = _gemv(1, k, n, 31)
    g4 = dict(_gemv(4, k, n, 31))
    g4["qd"], g4["sd"], g4["plane"] = g1["qd"], g1["sd"], g1["plane"]  # the same weight
    rc, staged = _prepare(g1["plane"], k, n)
    assert rc == 0, L.accel_hip_last_error()
    assert staged == STAGE_TILES | STAGE_GROUPS | STAGE_BF16 | STAGE_SMALL
    check(_call(g1))
    check(_call(g4))
    eager1, eager4 = g1["out"].numpy().copy(), g4["out"].numpy().copy()
    assert_gamma_bound(eager1, g1["a"], g1["w"])
    assert_gamma_bound(eager4, g4["a"], g1["w"])
    g1["out"].upload(np.zeros((1, n), np.float32))
    g4["out"].upload(np.zeros((4, n), np.float32))
    print("capture after prepare", flush=True)
    check(L.accel_hip_capture_begin())
    try:
        rc1, rc4 = _call(g1), _call(g4)
    finally:
        graph = _end_capture()
    try:
        assert (rc1, rc4) == (0, 0), L.accel_hip_last_error()
        scratch = dev(np.zeros(1024, np.float32))
        for rep in range(3):
            g1["out"].upload(np.zeros((1, n), np.float32))
            g4["out"].upload(np.zeros((4, n), np.float32))
            check(L.accel_hip_graph_launch(graph, 1))
            check(L.accel_hip_residual_add(scratch.buffer, scratch.buffer, 1024))  # eager work between replays
            same_bits(g1["out"].numpy(), eager1)
            same_bits(g4["out"].numpy(), eager4)
    finally:
        check(L.accel_hip_graph_destroy(graph))


def test_prepare_reports_and_refuses():
    """Layouts a plane cannot take are refused by name; a plane with zero points still gets
    its 8-column tiles; inside a capture the call is refused and enqueues nothing."""
    L = lib()
    k, n = 64, 96
    r = np.random.default_rng(5)
    q = dev(r.integers(-127, 128, size=k * n, dtype=np.int8))
    s = dev(r.uniform(1e-3, 1e-2, size=n).astype(np.float32))
    z = dev(r.integers(-3, 4, size=n, dtype=np.int8))
    plain = quant_plane(q, s, None, [k, n], 1)
    zero = quant_plane(q, s, z, [k, n], 1)
    assert _prepare(plain, k, n, STAGE_TILES) == (0, STAGE_TILES)
    assert _prepare(zero, k, n) == (0, STAGE_TILES)
    rc, _ = _prepare(zero, k, n, STAGE_GROUPS)
    assert rc == INVALID_ARGUMENT and b"group-interleaved" in L.accel_hip_last_error()
    rc, _ = _prepare(zero, k, n, STAGE_BF16)
    assert rc == INVALID_ARGUMENT and b"bf16 copy" in L.accel_hip_last_error()
    rc, _ = _prepare(zero, k, n, STAGE_SMALL)
    assert rc == INVALID_ARGUMENT and b"small GEMM" in L.accel_hip_last_error()
    rc, _ = _prepare(plain, 800, n, STAGE_SMALL)  # k > 768
    assert rc == INVALID_ARGUMENT
    rc, _ = _prepare(plain, k, n, 16)
    assert rc == INVALID_ARGUMENT and b"unknown layout" in L.accel_hip_last_error()
    rc, _ = _prepare(plain, 60, n, STAGE_GROUPS)  # k % 32 != 0
    assert rc == INVALID_ARGUMENT
    check(L.accel_hip_capture_begin())
    try:
        rc, staged = _prepare(plain, k, n)
        msg = L.accel_hip_last_error()
    finally:
        graph = _end_capture()
        check(L.accel_hip_graph_destroy(graph))
    assert rc == RUNTIME_ERROR and staged == 0, msg
    assert _prepare(plain, k, n) == (0, STAGE_TILES | STAGE_GROUPS | STAGE_BF16 | STAGE_SMALL)


def test_event_records_inside_a_capture_are_timeable():
    """accel_hip_event_record during a capture adds an event node that every replay records:
    the elapsed time between two such events is readable after each replay (a plain record
    inside a graph is refused by hipEventElapsedTime), positive, and no longer than the same
    replay timed from outside the graph (both spans from one replay: a replay's span varies
    with the clocks from one replay to the next)."""
    L = lib()
    g = _gemv(1, 1024, 4096, 91)
    check(_call(g))  # stage the weight copy eagerly
    check(L.accel_hip_synchronize())
    check(L.accel_hip_capture_begin())
    check(_call(g))
    check(L.accel_hip_event_record(0))
    for _ in range(5):
        check(_call(g))
    check(L.accel_hip_event_record(1))
    handle = _end_capture()
    try:
        for _ in range(3):
            check(L.accel_hip_event_record(2))
            check(L.accel_hip_graph_launch(handle, 1))
            check(L.accel_hip_event_record(3))
            outer = L.accel_hip_event_elapsed_ms(2, 3)
            assert outer > 0, L.accel_hip_last_error().decode()
            inner = L.accel_hip_event_elapsed_ms(0, 1)
            assert inner > 0, L.accel_hip_last_error().decode()
            assert inner <= outer
        np.testing.assert_allclose(g["out"].numpy(), g["a"].astype(np.float64) @ g["w"].astype(np.float64),
                                   rtol=1e-4, atol=1e-4)
    finally:
        check(L.accel_hip_graph_destroy(handle))


@pytest.mark.parametrize("m,k,n", [(128, 1024, 512), (64, 2048, 192)])
def test_fp32_weight_parts_staged_on_second_use(m, k, n):
    """The small-grid fp32 GEMM stages B as bf16 parts on B's second use with no write to it in
    between, and reads the parts from then on. The staged parts are the bits of the split on the
    fly, so every call stores the same bits. A graph captured after the staging reads the parts:
    rewriting B drops them and the graph is refused (which shows the parts were read). A B
    rewritten before each call (an activation) is never staged: its graph replays after the
    rewrite and follows the new values. (128 x 1024 x 512: one K range per workgroup; 64 x 2048 x
    192: K split over two workgroups.)"""
    L = lib()
    r = np.random.default_rng(m + n)
    a_h = r.standard_normal((m, k)).astype(np.float32)
    b1 = (r.standard_normal((k, n)) * 0.02).astype(np.float32)
    b2 = (r.standard_normal((k, n)) * 0.02).astype(np.float32)
    a, b, c = dev(a_h), dev(b1), dev(np.zeros((m, n), np.float32))

    def run():
        check(L.accel_hip_matmul_fused(a.ptr, b.ptr, c.ptr, m, k, n, None))
        return c.numpy()

    print(f"fp32 staged parts m={m} k={k} n={n}", flush=True)
    first = run()  # split on the fly; B seen once
    assert_gamma_bound(first, a_h, b1)
    same_bits(run(), first)  # stages the parts, then reads them
    same_bits(run(), first)
    check(L.accel_hip_capture_begin())
    try:
        check(L.accel_hip_matmul_fused(a.ptr, b.ptr, c.ptr, m, k, n, None))
    finally:
        graph = _end_capture()
    try:
        c.upload(np.zeros((m, n), np.float32))
        check(L.accel_hip_graph_launch(graph, 1))
        same_bits(c.numpy(), first)
        b.upload(b2)  # drops the staged parts the graph reads
        c.upload(np.full((m, n), 7.0, np.float32))
        rc = L.accel_hip_graph_launch(graph, 1)
        msg = L.accel_hip_last_error().decode()
        assert rc == RUNTIME_ERROR and "stale" in msg, (rc, msg)
        assert (c.numpy() == 7.0).all()  # nothing ran
    finally:
        check(L.accel_hip_graph_destroy(graph))
    again = run()  # seen again after the rewrite
    assert_gamma_bound(again, a_h, b2)
    same_bits(run(), again)  # staged anew

    # An activation: rewritten before every call, so never staged.
    act = dev(b1)
    outs = []
    for bh in (b1, b2, b1):
        act.upload(bh)
        check(L.accel_hip_matmul_fused(a.ptr, act.ptr, c.ptr, m, k, n, None))
        outs.append(c.numpy())
    same_bits(outs[0], first)
    same_bits(outs[1], again)
    same_bits(outs[2], first)
    check(L.accel_hip_capture_begin())
    try:
        check(L.accel_hip_matmul_fused(a.ptr, act.ptr, c.ptr, m, k, n, None))
    finally:
        graph = _end_capture()
    try:
        act.upload(b2)
        check(L.accel_hip_graph_launch(graph, 1))  # reads B itself: not stale
        same_bits(c.numpy(), again)
    finally:
        check(L.accel_hip_graph_destroy(graph))
