"""The C ABI of libcqgdn.so without a GPU: the library loads, exports every symbol include/cqgdn.h
declares, and its host-only functions (sizes, offsets, chunk table, argument checks) behave as
documented.  No call here launches a kernel."""

import ctypes
import re
from pathlib import Path

import pytest

from cqgdn import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "cqgdn.h"


def header_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(cqgdn_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built: run python cq-pretrain_amd/build.py")
    return _lib.lib()


def test_every_declared_symbol_is_exported_and_bound(lib):
    symbols = header_symbols()
    assert len(symbols) >= 15
    for name in symbols:
        assert hasattr(lib, name), f"{name} declared in cqgdn.h but not exported"
    assert set(symbols) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_version(lib):
    assert _lib.version().startswith("cqgdn ") and "gfx950" in _lib.version()


def test_header_constants_match_binding():
    text = HEADER.read_text()
    for name, value in (("CQGDN_FWD_BUFFERS", _lib.FWD_BUFFERS), ("CQGDN_BWD_BUFFERS", _lib.BWD_BUFFERS),
                        ("CQGDN_NORMALIZE", _lib.NORMALIZE), ("CQGDN_TRAINING", _lib.TRAINING),
                        ("CQGDN_PRECISE", _lib.PRECISE), ("CQGDN_NO_OUTPUT", _lib.NO_OUTPUT),
                        ("CQGDN_FP16", _lib.FP16), ("CQGDN_EINVAL", _lib.EINVAL), ("CQGDN_EUNSUPPORTED", _lib.EUNSUPPORTED),
                        ("CQGDN_EHIP", _lib.EHIP)):
        m = re.search(rf"#define {name} (\d+)", text)
        assert m and int(m.group(1)) == value, name


@pytest.mark.parametrize("T,H,nc", [(1, 4, 1), (129, 16, 3), (9216, 16, 144), (32768, 32, 530)])
def test_workspace_offsets_are_aligned_and_disjoint(lib, T, H, nc):
    for size_fn, offs_fn, n in ((lib.cqgdn_fwd_workspace_size, _lib.fwd_offsets, _lib.FWD_BUFFERS),
                                (lib.cqgdn_bwd_workspace_size, _lib.bwd_offsets, _lib.BWD_BUFFERS)):
        total = size_fn(T, H, nc)
        offs = list(offs_fn(T, H, nc).values())
        assert len(offs) == n and offs[0] == 0
        assert all(o % 256 == 0 for o in offs)
        # in order; the segment-map buffers are empty when no document has two segments
        assert all(b >= a for a, b in zip(offs, offs[1:])) and total >= offs[-1]
    # the largest per-chunk buffer is a [D][D] bf16 state per chunk and head
    offs = _lib.fwd_offsets(T, H, nc)
    assert offs["vnT"] - offs["hT"] >= nc * H * 128 * 128 * 2


def test_chunk_table_c_abi(lib):
    bounds = (ctypes.c_int64 * 4)(0, 10, 10, 140)
    n = lib.cqgdn_chunk_table(bounds, 4, None, None)
    assert n == 4
    table = (ctypes.c_int32 * (2 * n))()
    doc = (ctypes.c_int32 * 4)()
    assert lib.cqgdn_chunk_table(bounds, 4, table, doc) == n
    assert list(table) == [0, 10, 10, 64, 74, 64, 138, 2]
    assert list(doc) == [0, 1, 1, 4]
    bad = (ctypes.c_int64 * 3)(0, 10, 5)
    assert lib.cqgdn_chunk_table(bad, 3, None, None) == -1
    assert b"non-decreasing" in lib.cqgdn_last_error()


def _fwd(lib, **kw):
    p = ctypes.c_void_p(256)
    args = dict(q=p, k=p, v=p, g=p, beta=p, T=64, H=4, table=p, n_chunks=1, doc=p, n_docs=1, scale=0.1,
                flags=_lib.NORMALIZE | _lib.TRAINING, init=None, final=None, o=p, ws=p,
                ws_bytes=lib.cqgdn_fwd_workspace_size(64, 4, 1), stream=None)
    args.update(kw)
    return lib.cqgdn_fwd(*args.values())


def test_fwd_rejects_invalid_arguments_before_launch(lib):
    assert _fwd(lib, T=-1) == _lib.EINVAL
    assert _fwd(lib, H=0) == _lib.EINVAL
    assert _fwd(lib, n_chunks=0) == _lib.EINVAL
    assert _fwd(lib, q=None) == _lib.EINVAL
    assert _fwd(lib, ws_bytes=100) == _lib.EINVAL
    assert b"workspace" in lib.cqgdn_last_error()
    assert _fwd(lib, q=ctypes.c_void_p(258)) == _lib.EINVAL  # misaligned
    assert _fwd(lib, flags=_lib.PRECISE | _lib.TRAINING) == _lib.EINVAL
    assert b"PRECISE" in lib.cqgdn_last_error()
    assert _fwd(lib, flags=8) == _lib.EINVAL
    assert _fwd(lib, flags=32) == _lib.EINVAL and b"unknown flags" in lib.cqgdn_last_error()
    # fp16 inputs with either forward are valid requests: an invalid size still fails first
    for flags in (_lib.FP16 | _lib.TRAINING, _lib.FP16 | _lib.PRECISE, _lib.FP16):
        assert _fwd(lib, flags=flags | _lib.NORMALIZE, ws_bytes=100) == _lib.EINVAL
        assert b"workspace" in lib.cqgdn_last_error()


def test_bwd_checks_its_inputs_before_launch(lib):
    """The cached-mode backward reads q and k (the workspace keeps only their l2 scales), so
    they are checked like the other inputs; every case returns before the first HIP call."""
    p = ctypes.c_void_p(256)
    T, H, nc = 64, 4, 1

    def bwd(**kw):
        args = dict(q=p, k=p, v=p, g=p, beta=p, dout=p, T=T, H=H, table=p, n_chunks=nc, doc=p, n_docs=1, scale=0.1,
                    flags=_lib.NORMALIZE | _lib.TRAINING, fws=p, fws_bytes=lib.cqgdn_fwd_workspace_size(T, H, nc),
                    bws=p, bws_bytes=lib.cqgdn_bwd_workspace_size(T, H, nc), dq=p, dk=p, dv=p, dg=p, db=p,
                    stream=None)
        args.update(kw)
        return lib.cqgdn_bwd(*args.values())

    assert bwd(q=None) == _lib.EINVAL and b"null" in lib.cqgdn_last_error()
    assert bwd(k=None) == _lib.EINVAL
    assert bwd(k=ctypes.c_void_p(258)) == _lib.EINVAL and b"aligned" in lib.cqgdn_last_error()
    assert bwd(fws_bytes=100) == _lib.EINVAL and b"forward workspace" in lib.cqgdn_last_error()
    assert bwd(T=0, n_chunks=0) == _lib.OK  # nothing to do
    assert bwd(T=0, n_chunks=0, flags=_lib.NORMALIZE | _lib.TRAINING | _lib.FP16) == _lib.OK
    assert bwd(flags=_lib.NORMALIZE | _lib.TRAINING | _lib.FP16, q=None) == _lib.EINVAL
    assert bwd(flags=_lib.PRECISE) == _lib.EINVAL and b"unknown flags" in lib.cqgdn_last_error()


def _bwd_recompute(lib, **kw):
    p = ctypes.c_void_p(256)
    T, H, nc = kw.pop("T", 64), 4, 1
    args = dict(q=p, k=p, v=p, g=p, beta=p, dout=p, T=T, H=H, table=p, n_chunks=nc, doc=p, n_docs=1, scale=0.1,
                flags=_lib.NORMALIZE | _lib.TRAINING, fws=p, fws_bytes=lib.cqgdn_fwd_workspace_size(64, H, nc),
                bws=p, bws_bytes=lib.cqgdn_bwd_workspace_size(64, H, nc), dq=p, dk=p, dv=p, dg=p, db=p, stream=None)
    args.update(kw)
    return lib.cqgdn_bwd_recompute(*args.values())


def test_bwd_recompute_checks_every_argument_before_launch(lib):
    """The fused-mode backward (forward rebuilt in the same call) rejects bad arguments of either
    half before anything runs; every case here returns before the first HIP call."""
    assert _bwd_recompute(lib, flags=_lib.TRAINING | 8) == _lib.EINVAL  # CQGDN_NO_OUTPUT is implied, not a flag here
    assert _bwd_recompute(lib, T=-1) == _lib.EINVAL
    assert _bwd_recompute(lib, q=None) == _lib.EINVAL
    assert _bwd_recompute(lib, k=ctypes.c_void_p(258)) == _lib.EINVAL  # misaligned
    assert _bwd_recompute(lib, dq=None) == _lib.EINVAL
    assert _bwd_recompute(lib, bws_bytes=100) == _lib.EINVAL
    assert b"backward workspace" in lib.cqgdn_last_error()
    assert _bwd_recompute(lib, fws_bytes=100) == _lib.EINVAL
    assert _bwd_recompute(lib, T=0, n_chunks=0) == _lib.OK  # nothing to do


def test_recurrent_and_helpers_reject_invalid_arguments(lib):
    p = ctypes.c_void_p(256)
    assert lib.cqgdn_recurrent(p, p, p, p, p, 0, p, p, -1, 1, 4, 0.1, None) == _lib.EINVAL
    assert lib.cqgdn_recurrent(None, p, p, p, p, 0, p, p, 1, 1, 4, 0.1, None) == _lib.EINVAL
    assert lib.cqgdn_recurrent(p, p, p, p, p, 0, p, p, 0, 1, 4, 0.1, None) == _lib.OK  # nothing to do
    assert lib.cqgdn_recurrent(p, p, p, p, p, 4, p, p, 1, 1, 4, 0.1, None) == _lib.EINVAL  # unknown dtype flag
    assert lib.cqgdn_l2norm_fwd(p, p, None, -1, None) == _lib.EINVAL
    assert lib.cqgdn_l2norm_bwd(None, p, p, p, 4, None) == _lib.EINVAL
    assert lib.cqgdn_chunk_local_cumsum(None, p, 4, 4, p, 1, 0, None) == _lib.EINVAL


def test_timer_arguments(lib):
    assert lib.cqgdn_timer_arm(b"no_such_kernel", 4) == _lib.EINVAL
    assert lib.cqgdn_timer_arm(b"bwd_dkw", 0) == _lib.EINVAL
    assert lib.cqgdn_timer_arm(None, 0) == _lib.OK
    n = ctypes.c_int(-1)
    assert lib.cqgdn_timer_read(None, 0, ctypes.byref(n)) == _lib.OK and n.value == 0
    with pytest.raises(ValueError):
        _lib.KernelTimer("nope", 1)


def test_layer_decode_step_arguments(lib):
    # one launch and no workspace: the size is 0 and a NULL workspace is accepted
    assert lib.cqgdn_layer_decode_workspace_size(64, 16) == 0
    p = ctypes.c_void_p(256)
    w = ctypes.cast(p, ctypes.POINTER(ctypes.c_float))

    def step(N=1, H=16, HK=16, K=4, stride=4 * 16 * 128 + 32, ptr=p):
        return lib.cqgdn_layer_decode_step(N, H, HK, K, ptr, stride, p, p, w, w, w, 1e-6, 0.1, w, p, None, 0, None)

    assert step(N=0) == _lib.OK  # nothing to do, nothing launched
    assert step(H=12) == _lib.EINVAL
    assert step(HK=32) == _lib.EINVAL  # more key heads than value heads
    assert step(HK=2) == _lib.EINVAL
    # H = 32, key heads 8: C = (2 * 8 + 32) * 128 conv channels, then z (32 * 128), a and b (32 each)
    assert step(H=32, HK=8, stride=(16 + 64) * 128 + 64 - 8) == _lib.EINVAL
    assert b"proj_stride" in lib.cqgdn_last_error()
    assert step(N=0, H=32, HK=8) == _lib.OK
    assert step(K=5) == _lib.EINVAL
    assert step(stride=4 * 16 * 128) == _lib.EINVAL  # no room for the a, b columns
    assert b"proj_stride" in lib.cqgdn_last_error()
    assert step(ptr=ctypes.c_void_p(258)) == _lib.EINVAL  # misaligned projection rows


def test_training_forward_rejects_states(lib):
    """A CQGDN_TRAINING forward starts from a zero state and returns none (the reference's training
    adapter rejects both, ops/gated_delta_net.py:231-232); the check comes before any launch."""
    from cqgdn import _lib

    dummy = ctypes.c_void_p(16)
    rc = lib.cqgdn_fwd(dummy, dummy, dummy, dummy, dummy, 64, 4, dummy, 1, dummy, 1, 0.088, _lib.TRAINING, dummy, None,
                       dummy, dummy, 1 << 30, None)
    assert rc == _lib.EINVAL and b"zero state" in lib.cqgdn_last_error()


def test_torch_operators_are_registered():
    """libcqgdn_torch.so registers TORCH_LIBRARY(cqgdn) with the four per-step operators, whose schemas
    mark the decode state, the conv history and the decode output as written in place."""
    import torch

    ops = _lib.ops()
    schemas = {name: str(getattr(ops, name).default._schema)
               for name in ("fwd", "bwd", "recurrent", "layer_decode_step")}
    assert "Tensor? initial_state" in schemas["fwd"] and schemas["fwd"].endswith("-> (Tensor, Tensor, Tensor)")
    assert "Tensor? ws" in schemas["bwd"]
    assert "Tensor(a!) state, Tensor(b!) out" in schemas["recurrent"]
    assert "Tensor(a!) history, Tensor(b!) state" in schemas["layer_decode_step"]
    # CPU tensors are rejected with the reference's ValueError before anything runs
    q = torch.zeros(1, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm GPU"):
        ops.recurrent(q, q, q, torch.zeros(1, 4), torch.zeros(1, 4), torch.zeros(1, 4, 128, 128), q.clone(), 0.1)
