"""The C ABI of libxk_moe.so without a GPU: the library loads, it exports every
function include/xk_moe.h declares (and the ctypes table binds exactly those),
the pure-host size queries return the documented sizes, and argument checks
reject bad calls with XK_ERR_INVALID / XK_ERR_WORKSPACE before any HIP call."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from xkernels_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "xk_moe.h"


def _declared() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(xk_\w+)\s*\(", text))


def _defines() -> dict[str, int]:
    return {k: int(v) for k, v in re.findall(r"#define\s+(XK_\w+)\s+\(?(-?\d+)\)?", HEADER.read_text())}


def test_header_matches_binding_table():
    assert _declared() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing


def test_constants_match_header():
    d = _defines()
    for name in ("XK_OK", "XK_ERR_INVALID", "XK_ERR_WORKSPACE", "XK_ERR_LAUNCH", "XK_DT_BF16",
                 "XK_DT_FP32", "XK_DT_FP16", "XK_DT_NONE"):
        assert getattr(_lib, name) == d[name], name
    # the test-only kernel-choice bits live outside the public header
    internal = (_lib.ROOT_CSRC / "int4_flags.h").read_text()
    for name in ("XK_INT4_TEST_FORCE_TILE", "XK_INT4_TEST_FORCE_STREAM"):
        assert name not in d and name in internal
        assert getattr(_lib, "_" + name) == 1 << int(internal.split(name)[1].split("<<")[1].split(")")[0])


def test_version_and_empty_error():
    lib = _lib.load()
    assert lib.xk_abi_version() == 100
    assert isinstance(_lib.last_error(), str)


def _pad(numel, E, bs):
    return numel + (E + 1) * (bs - 1)


def test_size_queries():
    bs = _lib.query("xk_moe_int4_block_size", 64, 8, 48)
    assert bs >= 1
    assert _lib.query("xk_moe_int4_gemm_parts", 64, 8, 48, 4096, 7168, _lib.XK_DT_BF16, 32, 0) >= 1
    assert _lib.query("xk_moe_align_workspace_bytes", 512, 48) >= 0
    ws = _lib.query("xk_moe_int4_w4a16_workspace_bytes", 64, 8, 48, 4096, 7168)
    # at least the align outputs plus one fp32 row per routed slot
    assert ws >= 4 * (_pad(512, 48, bs) + 49) + 512 * 4096 * 4
    assert ws % 256 == 0
    wm = _lib.query("xk_moe_mxfp4_workspace_bytes", 48, 6, 256, 4096, 512)
    assert wm >= 288 * 512 * 2 + 288 * 4096 * 4


@pytest.mark.parametrize("E,hidden,ispp,top_k", [(256, 4096, 512, 6), (8, 256, 256, 2), (32, 512, 512, 4)])
def test_mxfp4_workspace_never_shrinks_with_batch(E, hidden, ispp, top_k):
    """A workspace sized for a batch must serve every smaller batch: the stream
    path cuts K into more slices for small batches, so its partial planes are
    sized for the largest slices x slots over the smaller sizes."""
    prev = 0
    for M in range(1, 70):
        b = _lib.query("xk_moe_mxfp4_workspace_bytes", M, top_k, E, hidden, ispp)
        assert b >= prev, (M, b, prev)
        prev = b


def _rc(name, *args):
    return getattr(_lib.load(), name)(*args)


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every case fails validation first


def test_align_rejects_bad_arguments():
    base = dict(ids=FAKE, numel=8, E=4, bs=4, emap=None, ng=0, s=FAKE, e=FAKE, n=FAKE, off=None,
                ws=FAKE, wsb=1 << 20, stream=None)

    def call(**kw):
        a = {**base, **kw}
        return _rc("xk_moe_align_block_size", a["ids"], a["numel"], a["E"], a["bs"], a["emap"], a["ng"],
                   a["s"], a["e"], a["n"], a["off"], a["ws"], a["wsb"], a["stream"])

    assert call(E=0) == _lib.XK_ERR_INVALID
    assert call(E=100000) == _lib.XK_ERR_INVALID
    assert "align" in _lib.last_error()
    assert call(bs=0) == _lib.XK_ERR_INVALID
    assert call(numel=-1) == _lib.XK_ERR_INVALID
    assert call(s=None) == _lib.XK_ERR_INVALID
    assert call(ids=None) == _lib.XK_ERR_INVALID
    assert call(emap=FAKE, ng=0) == _lib.XK_ERR_INVALID


def test_sum_reduce_rejects_bad_arguments():
    assert _rc("xk_moe_sum_reduce", FAKE, 7, 4, 2, 8, None, 0, 1.0, FAKE, None) == _lib.XK_ERR_INVALID
    assert _rc("xk_moe_sum_reduce", FAKE, 0, 4, 2, 8, FAKE, 9, 1.0, FAKE, None) == _lib.XK_ERR_INVALID
    assert _rc("xk_moe_sum_reduce", None, 0, 4, 2, 8, None, 0, 1.0, FAKE, None) == _lib.XK_ERR_INVALID
    assert _rc("xk_moe_sum_reduce", FAKE, 0, -1, 2, 8, None, 0, 1.0, FAKE, None) == _lib.XK_ERR_INVALID
    assert _rc("xk_moe_sum_reduce", FAKE, 0, 4, 2000, 8, None, 0, 1.0, FAKE, None) == _lib.XK_ERR_INVALID


def _int4(**kw):
    a = dict(A=FAKE, dt=0, M=4, K=64, packed=FAKE, scale=FAKE, E=2, N=16, gs=32, ids=FAKE, w=FAKE,
             k=2, emap=None, ng=0, mul=1, flags=0, out=FAKE, ws=FAKE, wsb=1 << 30, stream=None)
    a.update(kw)
    return _rc("xk_moe_int4_w4a16", a["A"], a["dt"], a["M"], a["K"], a["packed"], a["scale"], a["E"],
               a["N"], a["gs"], a["ids"], a["w"], a["k"], a["emap"], a["ng"], a["mul"], a["flags"],
               a["out"], a["ws"], a["wsb"], a["stream"])


def test_int4_rejects_bad_arguments():
    assert _int4(dt=5) == _lib.XK_ERR_INVALID
    assert _int4(k=0) == _lib.XK_ERR_INVALID
    assert _int4(out=None) == _lib.XK_ERR_INVALID
    assert _int4(packed=None) == _lib.XK_ERR_INVALID
    assert _int4(w=None) == _lib.XK_ERR_INVALID
    assert _int4(wsb=16) == _lib.XK_ERR_WORKSPACE
    assert "workspace" in _lib.last_error()
    assert _int4(ws=None) == _lib.XK_ERR_WORKSPACE
    assert _int4(M=0, A=None, out=None) == _lib.XK_OK  # empty batch: nothing to launch
    # flags: 0, or the test bits 8 / 9 (kernel choice); any other bit is rejected
    # before a launch, as is a test bit whose forced kernel needs more partial
    # planes than the workspace holds (covered on the GPU)
    assert _int4(flags=1) == _lib.XK_ERR_INVALID
    assert "flags" in _lib.last_error()
    assert _int4(flags=1 << 12) == _lib.XK_ERR_INVALID
    assert _int4(flags=1, M=0, A=None, out=None) == _lib.XK_ERR_INVALID
    # C5 shapes: the default choice (the tile kernel) writes one partial plane and
    # a workspace of the queried size holds one; forcing the stream kernel would
    # write two
    force_stream = _lib._XK_INT4_TEST_FORCE_STREAM
    nb = _lib.query("xk_moe_int4_w4a16_workspace_bytes", 4096, 8, 48, 4096, 7168)
    assert _int4(M=4096, K=7168, N=4096, E=48, k=8, flags=force_stream, wsb=nb) == _lib.XK_ERR_INVALID
    assert "partial planes" in _lib.last_error()


def test_int4_ep_workspace_covers_the_expert_parallel_choice():
    """Under an expert map the kernel choice counts the slots expected on the
    local experts: E = 48 local of 384 with 4096 slots is 10.7 rows per local
    expert (the decode stream kernel, 2 K-slice planes at K = 7168), where
    counting all slots would give 85 (the tile kernel, one plane). The expert
    workspace query sizes for the former; without a map it equals the dense one."""
    q = lambda *a: _lib.query("xk_moe_int4_w4a16_ep_workspace_bytes", *a)
    dense = lambda *a: _lib.query("xk_moe_int4_w4a16_workspace_bytes", *a)
    assert q(512, 8, 48, 4096, 7168, 0) == dense(512, 8, 48, 4096, 7168)
    assert q(512, 8, 48, 4096, 7168, 48) == dense(512, 8, 48, 4096, 7168)
    # C5 shapes (32768 slots): without a map fp32 activations take the scalar
    # kernel and bf16 the tile kernel (one plane each); 48 local experts of 2048
    # expect 16 rows each, where the bf16 choice is the stream kernel (two planes)
    plane = 32768 * 4096 * 4
    assert q(4096, 8, 48, 4096, 7168, 2048) - dense(4096, 8, 48, 4096, 7168) == plane
    assert q(4096, 8, 48, 4096, 7168, 96) == dense(4096, 8, 48, 4096, 7168)  # 341 rows: tile


def test_int4_kernel_choice_query():
    """Groups of 32, 64 and 128 take the MFMA kernels (decode stream below 17
    routed rows per expert, prefill tile from there, fp32 activations always
    the stream kernel) for K a multiple of 32 and N of 16; other shapes the
    scalar kernel."""
    k = lambda M, top_k, E, N, K, dt, gs, flags=0, ng=0: _lib.query(
        "xk_moe_int4_kernel", M, top_k, E, N, K, dt, gs, flags, ng)
    bf, f32 = _lib.XK_DT_BF16, _lib.XK_DT_FP32
    for gs in (32, 64, 128):
        assert k(64, 8, 48, 4096, 7168, bf, gs) == 1
        assert k(4096, 8, 48, 4096, 7168, bf, gs) == 2
        assert k(64, 8, 48, 4096, 7168, f32, gs) == 1
    assert k(64, 8, 48, 4096, 7168, bf, 256) == 0        # group size
    assert k(16, 8, 8, 512, 1344, bf, 64) == 1           # 21 scales a row (2-byte scale loads)
    assert k(16, 8, 8, 512, 1152, bf, 64) == 1           # 18 scales a row
    assert k(16, 2, 4, 48, 96, bf, 32) == 1              # K % 64 != 0, N % 32 != 0 (the spec's sweep point)
    assert k(16, 2, 4, 40, 96, bf, 32) == 0              # N % 16 != 0
    assert k(16, 2, 4, 48, 80, bf, 32) == 0              # K % 32 != 0
    assert k(4096, 8, 48, 4096, 7168, bf, 32, _lib._XK_INT4_TEST_FORCE_STREAM) == 1
    assert k(512, 8, 48, 4096, 7168, bf, 32, 0, 0) == 2    # 85 rows per expert
    assert k(512, 8, 48, 4096, 7168, bf, 32, 0, 384) == 1  # 10.7 expected per local expert
    # the MFMA kernels address A and one expert's weights through 32-bit buffer
    # offsets: past 2^31 bytes the call falls back to the scalar kernel
    assert k(149796, 8, 48, 4096, 7168, bf, 32) == 2     # A: 2^31 - 8,192 bytes
    assert k(149797, 8, 48, 4096, 7168, bf, 32) == 0     # A: 2^31 + 6,144 bytes
    assert k(256, 1, 1, 4096, 1048320, bf, 32) == 2      # one expert's weights just below 2^31 bytes
    assert k(256, 1, 1, 4096, 1048576, bf, 32) == 0      # 2^31 bytes


def test_int4_noalloc_rejects_unknown_flags():
    assert _rc("xk_moe_int4_w4a16_noalloc", FAKE, 0, 4, 64, FAKE, FAKE, 2, 16, 32, FAKE, FAKE, 2,
               None, 0, 1, 4, FAKE, None) == _lib.XK_ERR_INVALID


def test_int4_gemm_stage_rejects_bad_arguments():
    def g(**kw):
        a = dict(A=FAKE, dt=0, M=4, K=64, packed=FAKE, scale=FAKE, E=2, N=16, gs=32, ids=FAKE, k=2,
                 emap=None, ng=0, s=FAKE, off=FAKE, out=FAKE, flags=0, ws=None, wsb=0, stream=None)
        a.update(kw)
        return _rc("xk_moe_int4_w4a16_gemm", a["A"], a["dt"], a["M"], a["K"], a["packed"], a["scale"],
                   a["E"], a["N"], a["gs"], a["ids"], a["k"], a["emap"], a["ng"], a["s"], a["off"],
                   a["out"], a["flags"], a["ws"], a["wsb"], a["stream"])
    assert g(K=60) == _lib.XK_ERR_INVALID
    assert g(gs=48) == _lib.XK_ERR_INVALID
    assert g(dt=3) == _lib.XK_ERR_INVALID
    # flags: 0 is the only public value (the reference's bf16-rounded weights)
    assert g(flags=1) == _lib.XK_ERR_INVALID
    # the prefill tile kernel's queue: one counter per XCD
    assert _lib.query("xk_moe_int4_gemm_workspace_bytes", 4, 1024) == 32


def test_combine_rejects_bad_arguments():
    def c(**kw):
        a = dict(y=FAKE, M=4, k=2, N=16, w=FAKE, mul=1, ids=FAKE, nl=2, emap=None, ng=0, out=FAKE,
                 odt=0, parts=1, stream=None)
        a.update(kw)
        return _rc("xk_moe_topk_combine", a["y"], a["M"], a["k"], a["N"], a["w"], a["mul"], a["ids"],
                   a["nl"], a["emap"], a["ng"], a["out"], a["odt"], a["parts"], a["stream"])
    assert c(parts=0) == _lib.XK_ERR_INVALID
    assert c(parts=65) == _lib.XK_ERR_INVALID
    assert c(odt=4) == _lib.XK_ERR_INVALID
    assert c(w=None) == _lib.XK_ERR_INVALID
    assert c(k=0) == _lib.XK_ERR_INVALID


def _mx(**kw):
    a = dict(A=FAKE, dt=0, M=4, H=64, w13=FAKE, s13=FAKE, w2=FAKE, s2=FAKE, E=2, I=32, b13=None,
             b2=None, lim=7.0, gs=32, ids=FAKE, w=FAKE, k=2, emap=None, ng=0, mul=1, out=FAKE, ws=FAKE,
             wsb=1 << 30, stream=None)
    a.update(kw)
    return _rc("xk_moe_mxfp4", a["A"], a["dt"], a["M"], a["H"], a["w13"], a["s13"], a["w2"], a["s2"],
               a["E"], a["I"], a["b13"], a["b2"], a["lim"], a["gs"], a["ids"], a["w"], a["k"],
               a["emap"], a["ng"], a["mul"], a["out"], a["ws"], a["wsb"], a["stream"])


@pytest.mark.parametrize("kw,code", [
    (dict(gs=16), _lib.XK_ERR_INVALID), (dict(H=48), _lib.XK_ERR_INVALID),
    (dict(I=40), _lib.XK_ERR_INVALID), (dict(w2=None), _lib.XK_ERR_INVALID),
    (dict(dt=-1), _lib.XK_ERR_INVALID), (dict(w=None), _lib.XK_ERR_INVALID),
    (dict(wsb=100), _lib.XK_ERR_WORKSPACE), (dict(M=0, A=None, out=None), _lib.XK_OK),
])
def test_mxfp4_rejects_bad_arguments(kw, code):
    assert _mx(**kw) == code


def test_call_raises_with_message():
    with pytest.raises(RuntimeError, match="xk_moe_sum_reduce failed"):
        _lib.call("xk_moe_sum_reduce", FAKE, 7, 4, 2, 8, None, 0, 1.0, FAKE, None)


@pytest.mark.parametrize("kw", [dict(dt=3), dict(E=0), dict(E=(1 << 30) + 1, k=8), dict(k=0), dict(k=65),
                                dict(w=None), dict(ids=None), dict(g=None), dict(M=-1)])
def test_topk_softmax_rejects_bad_arguments(kw):
    a = dict(g=FAKE, dt=0, M=4, E=64, k=8, renorm=1, w=FAKE, ids=FAKE, stream=None)
    a.update(kw)
    assert _rc("xk_moe_topk_softmax", a["g"], a["dt"], a["M"], a["E"], a["k"], a["renorm"], a["w"],
               a["ids"], a["stream"]) == _lib.XK_ERR_INVALID
    assert "topk_softmax" in _lib.last_error()


def test_topk_softmax_empty_batch_is_ok():
    assert _rc("xk_moe_topk_softmax", None, 0, 0, 64, 8, 1, None, None, None) == _lib.XK_OK
