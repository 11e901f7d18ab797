"""The allocation-free matmul (jfh_engine_matmul_noalloc) against jfh_engine_matmul.

The no-alloc entry point takes device buffers and stages its int8 rows and
the fused device matrix's output rows in the library's static scratch; its
rows must equal the allocating entry point's bit for bit, on consecutive
calls that reuse the scratch (the second with fewer rows, so stale staging
from the first call would show), for a fused tensor of each layout kind, and
it rejects a call whose staging exceeds the scratch before doing any work. It
reads x after the work enqueued on the caller's stream: an input still being
copied there asynchronously is read complete.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import jetsonfabric_amd as jf
from jetsonfabric_amd._capi import check

pytestmark = pytest.mark.gpu

CFG = jf.ModelConfig(n_layer=1, n_embd=1024, n_ff=2816, n_head=8, n_head_kv=2, n_vocab=8192, n_ctx=256)
SCRATCH_BYTES = 16 << 20


class _Hip:
    """Device buffers for the test through the HIP runtime (the caller may allocate)."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so.7")

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed ({rc})")

    def upload(self, a: np.ndarray) -> ctypes.c_void_p:
        p = ctypes.c_void_p()
        self._ok(self.lib.hipMalloc(ctypes.byref(p), ctypes.c_size_t(a.nbytes)), "hipMalloc")
        self._ok(self.lib.hipMemcpy(p, a.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(a.nbytes), 1), "hipMemcpy")
        return p

    def alloc(self, nbytes: int) -> ctypes.c_void_p:
        p = ctypes.c_void_p()
        self._ok(self.lib.hipMalloc(ctypes.byref(p), ctypes.c_size_t(nbytes)), "hipMalloc")
        self._ok(self.lib.hipMemset(p, 0xFF, ctypes.c_size_t(nbytes)), "hipMemset")  # NaN fill: unwritten rows show
        return p

    def download(self, p: ctypes.c_void_p, shape) -> np.ndarray:
        out = np.zeros(shape, dtype=np.float32)
        self._ok(self.lib.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), p, ctypes.c_size_t(out.nbytes), 2),
                 "hipMemcpy")
        return out

    def free(self, p: ctypes.c_void_p) -> None:
        self.lib.hipFree(p)


@pytest.fixture(scope="module")
def engine():
    model = jf.Model.synthesize(CFG, type_linear=jf.Q4_K, type_embd=jf.Q4_K, type_output=jf.Q6_K, seed=23)
    e = jf.NativeEngine(model)
    yield e
    e.close()


def _noalloc(hip, engine, tensor, x, rows):
    xd = hip.upload(x)
    yd = hip.alloc(x.shape[0] * rows * 4)
    try:
        check(jf.library().jfh_engine_matmul_noalloc(engine.handle, tensor.encode(), xd, x.shape[0], yd, None))
        return hip.download(yd, (x.shape[0], rows))
    finally:
        hip.free(xd)
        hip.free(yd)


# tensor -> (rows, cols): q (RoPE pair order inside the fused qkv), v (plain
# rows of qkv), gate / up (interleaved GLU rows), down, and the Q6_K head
TENSORS = {
    "blk.0.attn_q.weight": (1024, 1024),
    "blk.0.attn_v.weight": (256, 1024),
    "blk.0.ffn_gate.weight": (2816, 1024),
    "blk.0.ffn_up.weight": (2816, 1024),
    "blk.0.ffn_down.weight": (1024, 2816),
    "output.weight": (8192, 1024),
}


@pytest.mark.parametrize("tensor", list(TENSORS))
def test_noalloc_matmul_equals_the_allocating_one(engine, tensor):
    hip = _Hip()
    rows, cols = TENSORS[tensor]
    rng = np.random.default_rng(sum(tensor.encode()))
    # a wide call, then a smaller one (token quads), then one row (decode matmul)
    for n_tok in (40, 5, 1):
        x = rng.normal(0, 1, (n_tok, cols)).astype(np.float32)
        want = engine.matmul(tensor, x, rows)
        got = _noalloc(hip, engine, tensor, x, rows)
        assert np.array_equal(got, want), f"{tensor} n_tok {n_tok}: max diff {np.abs(got - want).max()}"


def test_noalloc_rejects_staging_beyond_the_scratch(engine):
    hip = _Hip()
    # the head's full output rows for 256 tokens (the row limit): 256 x 8192 x 4 B = 8 MiB fits; a larger
    # model's would not, so ask for more rows than the scratch holds through the widest tensor the engine has
    rows, cols = TENSORS["output.weight"]
    n_tok = 256
    need = n_tok * rows * 4
    assert need <= SCRATCH_BYTES  # this engine's largest call fits
    x = np.zeros((n_tok, cols), dtype=np.float32)
    got = _noalloc(hip, engine, "output.weight", x, rows)
    assert np.array_equal(got, engine.matmul("output.weight", x, rows))
    # a call beyond the engine's row limit is rejected before any work
    with pytest.raises(jf.JfhError):
        _noalloc(hip, engine, "output.weight", np.zeros((257, cols), dtype=np.float32), rows)


def test_noalloc_rejects_a_call_larger_than_the_scratch():
    """A vocabulary large enough that the head's staging for 64 rows exceeds
    16 MiB: the call fails with an invalid-argument status and names the limit."""
    cfg = jf.ModelConfig(n_layer=1, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=70000, n_ctx=64)
    model = jf.Model.synthesize(cfg, type_linear=jf.Q4_K, type_embd=jf.Q4_K, type_output=jf.Q4_K, seed=3)
    e = jf.NativeEngine(model)
    hip = _Hip()
    try:
        x = np.zeros((64, 256), dtype=np.float32)
        with pytest.raises(jf.JfhError, match="static scratch holds 16777216"):
            _noalloc(hip, e, "output.weight", x, 70000)
        # the same tensor over 8 rows fits and matches
        x8 = np.random.default_rng(1).normal(0, 1, (8, 256)).astype(np.float32)
        assert np.array_equal(_noalloc(hip, e, "output.weight", x8, 70000), e.matmul("output.weight", x8, 70000))
    finally:
        e.close()


def test_noalloc_reads_x_after_the_callers_stream(engine):
    """x is written by an asynchronous copy from pinned memory on the caller's
    non-blocking stream and the matmul is called at once with that stream: the
    result equals the allocating matmul's on the same rows, bit for bit."""
    hip = _Hip()
    lib = hip.lib
    tensor = "blk.0.ffn_down.weight"
    rows, cols = TENSORS[tensor]
    stream = ctypes.c_void_p()
    hip._ok(lib.hipStreamCreateWithFlags(ctypes.byref(stream), 1), "hipStreamCreateWithFlags")
    n_tok = 16
    nbytes = n_tok * cols * 4
    pinned = ctypes.c_void_p()
    hip._ok(lib.hipHostMalloc(ctypes.byref(pinned), ctypes.c_size_t(nbytes), 0), "hipHostMalloc")
    xd = hip.alloc(nbytes)  # NaN-filled: a matmul that ran ahead of the copy would read them
    yd = hip.alloc(n_tok * rows * 4)
    try:
        rng = np.random.default_rng(77)
        for it in range(3):
            x = rng.normal(0, 1, (n_tok, cols)).astype(np.float32)
            ctypes.memmove(pinned, x.ctypes.data, nbytes)
            hip._ok(lib.hipMemsetAsync(xd, 0xFF, ctypes.c_size_t(nbytes), stream), "hipMemsetAsync")
            hip._ok(lib.hipMemcpyAsync(xd, pinned, ctypes.c_size_t(nbytes), 1, stream), "hipMemcpyAsync")
            check(jf.library().jfh_engine_matmul_noalloc(engine.handle, tensor.encode(), xd, n_tok, yd, stream))
            got = hip.download(yd, (n_tok, rows))
            assert np.array_equal(got, engine.matmul(tensor, x, rows)), f"call {it}"
    finally:
        hip._ok(lib.hipStreamSynchronize(stream), "hipStreamSynchronize")
        hip.free(xd)
        hip.free(yd)
        lib.hipHostFree(pinned)
        lib.hipStreamDestroy(stream)
