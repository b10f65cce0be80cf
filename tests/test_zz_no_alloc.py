"""cqgdn_fwd_static, the forward that allocates nothing (include/cqgdn.h), through the C ABI.

It must give exactly what cqgdn_fwd gives with a caller workspace (same kernels, same inputs; bf16
and fp16 q/k/v), on two calls in a row -- the second smaller, so it runs over what the first left in the shared
static workspace -- leave the device's free memory unchanged once cqgdn_fwd_static_init has reserved
the static array on the device (a second set-up reserves nothing more), replay from a HIP graph it was captured into with the results of
the eager call, and reject what it cannot serve: a workspace larger than its static one, and a
training forward."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _run(gdn, lib, xs, bounds, static, initial_state=None, free_bytes=None):
    from cqgdn import _lib

    q, k, v, g, b = (x.to(DEV).contiguous() for x in xs)
    T, H = q.shape[1], q.shape[2]
    _, table, doc = gdn.device_metadata(bounds, DEV)
    nc, nd = table.shape[0], len(bounds) - 1
    o = torch.empty_like(v)
    state = torch.empty(nd, H, 128, 128, dtype=torch.float32, device=DEV)
    init = None if initial_state is None else initial_state.to(DEV).contiguous()
    flags = _lib.NORMALIZE | _lib.PRECISE | (_lib.FP16 if q.dtype == torch.float16 else 0)
    P = gdn._ptr
    common = (P(q), P(k), P(v), P(g), P(b), T, H, P(table), nc, P(doc), nd, 128 ** -0.5, flags, P(init), P(state),
              P(o))
    if static:
        torch.cuda.synchronize()
        before = torch.cuda.mem_get_info()[0]
        rc = lib.cqgdn_fwd_static(*common, gdn._stream(q.device))
        torch.cuda.synchronize()
        if free_bytes is not None:
            free_bytes.append((before, torch.cuda.mem_get_info()[0]))
    else:
        ws = torch.empty(lib.cqgdn_fwd_workspace_size(T, H, nc), dtype=torch.uint8, device=DEV)
        rc = lib.cqgdn_fwd(*common, P(ws), ws.numel(), gdn._stream(q.device))
    assert rc == 0, lib.cqgdn_last_error().decode()
    torch.cuda.synchronize()
    return o, state


def test_static_forward_matches_workspace_forward(gdn):
    from cqgdn import _lib, synthetic

    lib = _lib.lib()
    torch.cuda.synchronize()
    before = torch.cuda.mem_get_info()[0]
    assert lib.cqgdn_fwd_static_init() == 0, lib.cqgdn_last_error().decode()
    torch.cuda.synchronize()
    middle = torch.cuda.mem_get_info()[0]
    # the first set-up in a process may also have the runtime load the library's other code objects
    print(f"  set-up reserved {before - middle} bytes (static array {_lib.STATIC_WORKSPACE_BYTES})", flush=True)
    assert lib.cqgdn_fwd_static_init() == 0, lib.cqgdn_last_error().decode()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == middle, "a second set-up reserved memory again"
    # each second call smaller than the one before it; then the same with fp16 q/k/v (CQGDN_FP16)
    cases = [(1900, (0, 700, 1900), 16, None, torch.bfloat16), (300, (0, 129, 300), 16, 0.05, torch.bfloat16),
             (1200, (0, 500, 1200), 16, 0.05, torch.float16), (257, (0, 257), 16, None, torch.float16)]
    for T, bounds, H, s0, dtype in cases:
        print(f"case static forward T={T} bounds={bounds} H={H} {dtype}", flush=True)
        xs = [x.to(dtype) if x.dim() == 4 else x for x in synthetic.make_inputs(T, H, 128, seed=T)]
        init = None if s0 is None else torch.randn(len(bounds) - 1, H, 128, 128,
                                                   generator=torch.Generator().manual_seed(5)) * s0
        o_ws, st_ws = _run(gdn, lib, xs, bounds, False, init)
        free = []
        o_st, st_st = _run(gdn, lib, xs, bounds, True, init, free)
        print(f"  free device bytes around the static call: {free[0][0]} -> {free[0][1]}", flush=True)
        assert free[0][0] == free[0][1], "the static forward changed the device's free memory"
        assert torch.equal(o_ws, o_st)
        assert torch.equal(st_ws, st_st)
        assert torch.isfinite(o_st.float()).all()


def test_static_forward_replays_in_a_hip_graph(gdn):
    """cqgdn_fwd_static captured into a HIP graph (no allocation and no memset inside the call, so it
    captures as plain kernel nodes): four replays, with eager work and synchronizations between them
    (a workspace forward of other inputs that runs over the same kernels), each equal to the eager
    static call."""
    from cqgdn import _lib, synthetic

    lib = _lib.lib()
    assert lib.cqgdn_fwd_static_init() == 0, lib.cqgdn_last_error().decode()
    T, bounds, H = 700, (0, 250, 700), 16
    print(f"case static forward in a graph T={T} bounds={bounds} H={H}", flush=True)
    xs = [x.to(DEV).contiguous() for x in synthetic.make_inputs(T, H, 128, seed=77)]
    other = synthetic.make_inputs(T, H, 128, seed=78)
    _, table, doc = gdn.device_metadata(bounds, DEV)
    nc, nd = table.shape[0], len(bounds) - 1
    o = torch.empty_like(xs[2])
    state = torch.empty(nd, H, 128, 128, dtype=torch.float32, device=DEV)
    P = gdn._ptr

    def call():
        q, k, v, g, b = xs
        rc = lib.cqgdn_fwd_static(P(q), P(k), P(v), P(g), P(b), T, H, P(table), nc, P(doc), nd, 128 ** -0.5,
                                  _lib.NORMALIZE | _lib.PRECISE, None, P(state), P(o),
                                  torch.cuda.current_stream().cuda_stream)
        assert rc == 0, lib.cqgdn_last_error().decode()

    call()
    torch.cuda.synchronize()
    o_eager, st_eager = o.clone(), state.clone()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for replay in range(4):
        o.zero_()
        state.zero_()
        _run(gdn, lib, other, bounds, False)  # eager work over the same kernels between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_eager), f"replay {replay}: output differs from the eager call"
        assert torch.equal(state, st_eager), f"replay {replay}: final state differs from the eager call"


def test_static_forward_rejects_what_it_cannot_serve(gdn):
    from cqgdn import _lib, synthetic

    lib = _lib.lib()
    T, H = 4096, 16  # needs more than the 64 MiB static workspace
    q, k, v, g, b = (x.to(DEV) for x in synthetic.make_inputs(T, H, 128, seed=1))
    _, table, doc = gdn.device_metadata((0, T), DEV)
    o = torch.empty_like(v)
    P = gdn._ptr
    assert lib.cqgdn_fwd_workspace_size(T, H, table.shape[0]) > _lib.STATIC_WORKSPACE_BYTES
    rc = lib.cqgdn_fwd_static(P(q), P(k), P(v), P(g), P(b), T, H, P(table), table.shape[0], P(doc), 1,
                              128 ** -0.5, _lib.NORMALIZE | _lib.PRECISE, None, None, P(o), None)
    assert rc == _lib.EINVAL and b"static one" in lib.cqgdn_last_error()
    rc = lib.cqgdn_fwd_static(P(q), P(k), P(v), P(g), P(b), 64, H, P(table), 1, P(doc), 1, 128 ** -0.5,
                              _lib.NORMALIZE | _lib.TRAINING, None, None, P(o), None)
    assert rc == _lib.EINVAL and b"TRAINING" in lib.cqgdn_last_error()
