"""C ABI: the library loads, exports every symbol include/w4a8_amd.h declares,
and rejects bad arguments on the host (before any launch, so these run
without a GPU)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "w4a8_amd.h"


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(w4a8_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg._abi.lib()


def test_header_symbols_are_exported(pkg, lib):
    syms = declared_symbols()
    assert len(syms) >= 9
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in {HEADER.name} but not exported"
        assert s in pkg._abi.SIGNATURES, f"{s} has no ctypes signature"


def test_version_and_sizes(lib):
    assert lib.w4a8_abi_version() == 10
    # 16-column x 128-K tiles of 1 KB; scales [ceil(N/16), G, 16] x 2 bytes
    assert lib.w4a8_repacked_weight_bytes(5120, 5120, 128) == 320 * 40 * 1024
    assert lib.w4a8_repacked_weight_bytes(100, 512, 64) == 7 * 4 * 1024
    assert lib.w4a8_repacked_scale_bytes(100, 512, 64) == 7 * 8 * 16 * 2
    assert lib.w4a8_repacked_weight_bytes(0, 512, 64) == -1
    # prefill and most decode shapes need no workspace; past 8 rows on narrow
    # N with long K (>= 128 tiles) the decode GEMM splits K over workgroups
    # and keeps fp32 sums [splits, M, ceil(N/16)*16] there
    assert lib.w4a8_gemm_workspace_bytes(4096, 5120, 5120, 128) == 0
    assert lib.w4a8_gemm_workspace_bytes(16, 5120, 5120, 128) == 0
    assert lib.w4a8_gemm_workspace_bytes(8, 5120, 27648, 128) == 0
    assert lib.w4a8_gemm_workspace_bytes(64, 5120, 27648, 128) == 6 * 64 * 5120 * 4
    assert lib.w4a8_gemm_workspace_bytes(48, 5120, 27648, 128) == 6 * 48 * 5120 * 4   # split 64-row prefill tile
    assert lib.w4a8_gemm_workspace_bytes(24, 5120, 27648, 128) == 8 * 24 * 5120 * 4
    assert lib.w4a8_gemm_workspace_bytes(12, 5120, 27648, 128) == 12 * 12 * 5120 * 4
    assert lib.w4a8_gemm_workspace_bytes(20, 1000, 16384, 128) == 16 * 20 * 1008 * 4
    assert lib.w4a8_gemm_workspace_bytes(64, 55296, 27648, 128) == 0   # wide N: no split


def _gemm(lib, **kw):
    a = dict(a_q=16, lda=256, a_scale=16, w_tiles=16, s_tiles=16, sd=0, y=16, ldy=64, M=4, N=64, K=256,
             group=128, ws=None, wsb=0)
    a.update(kw)
    return lib.w4a8_gemm(a["a_q"], a["lda"], a["a_scale"], a["w_tiles"], a["s_tiles"], a["sd"], a["y"],
                         a["ldy"], a["M"], a["N"], a["K"], a["group"], a["ws"], a["wsb"], None)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(N=0), 2, "bad shape"),
    (dict(M=-1), 2, "bad shape"),
    (dict(K=300), 2, "kpad=320"),               # ragged K: A is read in the padded layout
    (dict(group=96, K=192, lda=240), 2, "kpad=256"),  # groups padded to 128 each
    (dict(sd=7), 3, "scale_dtype"),
    (dict(a_q=None), 1, "NULL"),
    (dict(lda=100), 2, "lda"),
    (dict(lda=264), 4, "16-byte"),
    (dict(a_q=24), 4, "16-byte"),
    # the wide decode layouts read two columns' scales as one dword
    (dict(s_tiles=18), 4, "s_tiles 4-byte aligned"),
    # a decode shape that splits K over workgroups needs its workspace
    (dict(M=12, N=5120, K=27648, lda=27648, ldy=5120), 6, "workspace needs 2949120 bytes"),
    (dict(M=12, N=5120, K=27648, lda=27648, ldy=5120, ws=256, wsb=2949119), 6, "workspace"),
    (dict(M=12, N=5120, K=27648, lda=27648, ldy=5120, ws=272, wsb=1 << 21), 6, "256-byte aligned"),
])
def test_gemm_rejects_bad_arguments(lib, kw, code, msg):
    # Fake, never-dereferenced addresses: validation fails before any launch.
    assert _gemm(lib, **kw) == code
    assert msg in lib.w4a8_last_error().decode()


def test_stream_capture_id_rejects_null_and_idle_streams(lib):
    assert lib.w4a8_stream_capture_id(None, None) == 1
    # the null stream is never being captured; on a host without a GPU the
    # runtime query itself fails, which is reported as a HIP error
    cid = ctypes.c_ulonglong(0)
    assert lib.w4a8_stream_capture_id(None, ctypes.byref(cid)) in (5, 7)


def test_m0_is_a_noop(lib):
    assert _gemm(lib, M=0, a_q=None, y=None) == 0


def test_quant_and_repack_reject_bad_arguments(lib):
    assert lib.w4a8_quant_act(None, 64, None, 64, None, 4, 64, 0, None) == 1
    assert lib.w4a8_quant_act(16, 32, 16, 64, 16, 4, 64, 0, None) == 2
    assert lib.w4a8_quant_act(None, 64, None, 64, None, 0, 64, 0, None) == 0
    # the padded layout of K=100, group 33 is 4 * 64 = 256 wide
    assert lib.w4a8_quant_act(16, 128, 16, 128, 16, 4, 100, 33, None) == 2
    assert "output width 256" in lib.w4a8_last_error().decode()
    assert lib.w4a8_quant_act(16, 128, 16, 256, 16, 4, 100, -1, None) == 2
    assert lib.w4a8_repack(16, 16, 2, 16, 16, 64, 256, 128, None) == 3
    assert lib.w4a8_repack(18, 16, 0, 16, 16, 64, 256, 128, None) == 4
    assert lib.w4a8_repack(16, 16, 0, 16, 16, 64, 256, 0, None) == 2


def test_rope_kv_rejects_bad_arguments(lib):
    # fake, never-dereferenced addresses: validation fails before any launch
    st = (ctypes.c_int64 * 4)(1, 1, 1, 1)

    def call(**kw):
        a = dict(qkv=16, ldq=7168, cos=16, sin=16, ldc=64, L=64, pos=16, q=16, kc=16, vc=16, B=1, T=1, H=40,
                 KVH=8, D=128)
        a.update(kw)
        return lib.w4a8_rope_kv(a["qkv"], a["ldq"], a.get("bias"), a["cos"], a["sin"], a["ldc"], a["L"], a["pos"],
                                a["q"], a["kc"], st, a["vc"], st, a["B"], a["T"], a["H"], a["KVH"], a["D"], None)
    assert call(D=127) == 2 and "D even" in lib.w4a8_last_error().decode()
    assert call(L=0) == 2
    assert call(ldq=7000) == 2 and "leading dimensions" in lib.w4a8_last_error().decode()
    assert call(ldc=63) == 2
    assert call(qkv=None) == 1
    assert call(cos=18) == 4                 # fp32 table not 4-byte aligned
    assert call(pos=20) == 4                 # int64 position not 8-byte aligned
    assert call(bias=17) == 4                # bf16 bias not 2-byte aligned
    assert call(H=65535) == 2                # one workgroup row per head
    assert call(B=0, qkv=None) == 0          # nothing to do
    assert lib.w4a8_rope_kv(16, 7168, None, 16, 16, 64, 64, 16, 16, 16, None, 16, st, 1, 1, 40, 8, 128, None) == 1


def test_errors_raise_runtimeerror_from_python(pkg):
    with pytest.raises(RuntimeError, match="SHAPE"):
        pkg._abi.check(_gemm(pkg._abi.lib(), N=0), "w4a8_gemm")


def test_row_chunk_arithmetic(lib):
    """Calls whose activations exceed 32-bit offsets are split into row chunks: each
    chunk fits the offset bound (rows + 128 past them), chunks are multiples of 128,
    and a balanced split of M gives every chunk more than 64 rows (prefill launches)."""
    for lda in (5120, 27648, 55296, 1 << 16, 1 << 20, 3 << 20):
        for M in (1, 64, 65, 1000, 77000, 77700, 80000, 200000, 1 << 20):
            c = lib.w4a8_gemm_row_chunk(M, lda)
            if (M + 128) * lda < (1 << 31):
                assert c == M
                continue
            if M <= 64:
                assert c == 0
                continue
            if c == 0:
                assert ((1 << 31) - 1) // lda - 128 < 256
                continue
            assert c % 128 == 0 and c >= 256 and (c + 128) * lda < (1 << 31)
            n = -(-M // c)
            bounds = [(M * i) // n for i in range(n + 1)]
            sizes = [b - a for a, b in zip(bounds, bounds[1:])]
            assert sum(sizes) == M and max(sizes) <= c and min(sizes) > 64
    assert lib.w4a8_gemm_row_chunk(80000, 27648) == ((1 << 31) - 1) // 27648 - 128 - (((1 << 31) - 1) // 27648 - 128) % 128


def test_offset_limits_are_refused_on_every_path(lib):
    """Weights beyond 32-bit offsets are refused by the GEMM and by the fused
    single-row linear alike (no launch, no silent wrap)."""
    N, K, G = 1 << 19, 8192, 128
    st = lib.w4a8_gemm(16, K, 16, 16, 16, 0, 16, N, 1, N, K, G, None, 0, None)
    assert st == 5 and b"32-bit" in lib.w4a8_last_error()
    st = lib.w4a8_linear(16, K, 16, 16, 0, 16, N, 16, K, 16, 1, N, K, G, None, 0, None)
    assert st == 5 and b"32-bit" in lib.w4a8_last_error()
    # 64 rows at a stride too large for one launch cannot be chunked
    lda = (1 << 31) // 150 // 16 * 16
    assert lib.w4a8_gemm(16, lda, 16, 16, 16, 0, 16, 64, 64, 64, 256, G, None, 0, None) == 5


def test_attention_sizes_and_rejects_bad_arguments(lib):
    # decode splits (256 CUs assumed without a GPU): 8 row tiles split 8 ways (3 chunks
    # each), 64 tiles 4 ways, 512 tiles (one per CU at least) not at all; a long
    # cache of one sequence into up to Lc / 1024 splits
    assert lib.w4a8_attention_chunks_per_split(1, 40, 8, 1280) == 3
    assert lib.w4a8_attention_chunks_per_split(8, 40, 8, 1280) == 5
    assert lib.w4a8_attention_chunks_per_split(64, 40, 8, 1280) == 20
    assert lib.w4a8_attention_chunks_per_split(1, 40, 8, 32768) == 16
    assert lib.w4a8_attention_chunks_per_split(1, 40, 8, 1000) == -1      # cache axis not a multiple of 64
    assert lib.w4a8_attention_chunks_per_split(1, 40, 7, 1280) == -1      # H not a multiple of KVH
    # workspace: one state of D + 4 floats per row and split, none with a single split
    assert lib.w4a8_attention_workspace_bytes(2, 1, 40, 128, 1280, 5) == 2 * 40 * 4 * 132 * 4
    assert lib.w4a8_attention_workspace_bytes(2, 1, 40, 128, 1280, 3) == 2 * 40 * 7 * 132 * 4
    assert lib.w4a8_attention_workspace_bytes(2, 1, 40, 128, 1280, 20) == 0

    def call(**kw):
        a = dict(q=16, k=16, vt=16, out=16, pos=16, B=1, T=1, H=40, KVH=8, D=128, L=1280, Lc=1280, cps=1,
                 scale=0.088, ws=None, wsb=0)
        a.update(kw)
        return lib.w4a8_attention(a["q"], a["k"], a["vt"], a["out"], a["pos"], a["B"], a["T"], a["H"], a["KVH"],
                                  a["D"], a["L"], a["Lc"], a["cps"], a["scale"], a["ws"], a["wsb"], None)
    assert call(D=96) == 5 and b"64 or 128" in lib.w4a8_last_error()
    assert call(KVH=7) == 2
    assert call(Lc=1000) == 2 and b"multiple of 64" in lib.w4a8_last_error()
    assert call(L=1300) == 2
    assert call(cps=21) == 2 and b"chunks_per_split" in lib.w4a8_last_error()
    assert call(scale=float("inf")) == 2
    assert call(q=None) == 1
    assert call(k=24) == 4
    assert call(ws=16, wsb=100) == 6 and b"workspace needs" in lib.w4a8_last_error()
    assert call(B=0, q=None) == 0


def test_attention_rope_rejects_bad_arguments(lib):
    def call(**kw):
        a = dict(qkv=16, ldq=7168, bias=None, cos=16, sin=16, ldc=64, k=16, vt=16, out=16, pos=16, B=1, H=40, KVH=8,
                 D=128, L=1280, Lc=1280, cps=3, scale=0.088, ws=16, wsb=1 << 20)
        a.update(kw)
        return lib.w4a8_attention_rope(a["qkv"], a["ldq"], a["bias"], a["cos"], a["sin"], a["ldc"], a["k"], a["vt"],
                                       a["out"], a["pos"], a["B"], a["H"], a["KVH"], a["D"], a["L"], a["Lc"],
                                       a["cps"], a["scale"], a["ws"], a["wsb"], None)
    assert call(qkv=None) == 1
    assert call(ldq=7000) == 2 and b"ldq" in lib.w4a8_last_error()
    assert call(ldc=63) == 2
    assert call(qkv=24) == 4                        # qkv rows read 16 bytes at a time
    assert call(cos=18) == 4
    assert call(ws=None, wsb=0) == 6                # 7 splits: the combine needs its workspace
    assert call(D=96, ldq=96 * 56) == 5


def test_midgroup_workspace_sizes_and_rejects(lib):
    """The compat GEMM's prefill path: its workspace query (rebuilt activation rows
    [Ma, k_tiles * 128] and fp32 activation scales [G, Ma], then from 1024 rows the
    repacked weight tiles, each 256-byte aligned; 0 where the mid-group kernel runs) and
    the host checks of w4a8_midgroup_gemm_ws, before any launch.  Without a GPU the
    library takes 256 CUs."""
    q = lib.w4a8_midgroup_gemm_workspace_bytes
    c256 = lambda n: -(-n // 256) * 256
    tiled = c256(c256(4096 * 5120) + 5 * 4096 * 4) + 448 * 40 * 1024
    assert q(4096, 7168, 5120, 1024) == tiled
    assert q(4096, 7168, 5000, 1000) == tiled                    # stride 1024, ragged K
    assert q(100, 8192, 1057, 1024) == c256(100 * 1152) + 2 * 100 * 4
    assert q(65, 8200, 3456, 256) == c256(65 * 3456) + 14 * 65 * 4
    assert q(1000, 7168, 5120, 1024) == c256(1000 * 5120) + 5 * 1000 * 4
    assert q(1024, 7168, 5120, 1024) == c256(c256(1024 * 5120) + 5 * 1024 * 4) + 448 * 40 * 1024
    # wide N from 17 rows (one row tile of 432 column tiles)
    assert q(17, 55296, 5120, 1024) == c256(17 * 5120) + 5 * 17 * 4
    assert q(64, 55296, 5120, 1024) == c256(64 * 5120) + 5 * 64 * 4
    # the mid-group kernel keeps: up to 16 rows, 64-row tiles for fewer than half
    # the CUs, group stride 128 or not a multiple of 128, offsets past 2^31
    assert q(16, 55296, 5120, 1024) == 0
    assert q(64, 7168, 5120, 1024) == 0
    assert q(128, 7168, 5120, 1024) == 0 and q(256, 7168, 5120, 1024) > 0
    assert q(4096, 7168, 5120, 128) == 0
    assert q(4096, 7168, 5120, 64) == 0
    assert q(80000, 5120, 27648, 1024) == 0
    assert q(0, 512, 1024, 1024) == 0 and q(100, 0, 1024, 1024) == 0 and q(100, 512, 1024, 0) == 0

    def call(ws, wsb, Ma=128, ld_as=128):
        return lib.w4a8_midgroup_gemm_ws(16, 16, 16, 16, Ma, ld_as, 16, 16, 16, 16, 16384, None, 16384, 2048, 1024,
                                         ws, wsb, None)
    need = q(128, 16384, 2048, 1024)
    assert need > 0
    assert call(None, need) == 6 and b"workspace" in lib.w4a8_last_error()
    assert call(4096, need - 1) == 6
    assert call(4096 + 16, need) == 6                 # not 256-byte aligned
    assert call(4096, -1) == 6
    assert call(4096, need, ld_as=64) == 2            # ld_as < rows


def test_midgroup_group_count_limit(lib):
    """The compat kernel stages every group's row and column values in at most 128 KiB of
    LDS (16-row tiles where 64 rows' values do not fit: about 330 groups): 782 groups at
    K=100000, group 128 are refused before any launch, at one row and at 64."""
    for Ma in (1, 64):
        rc = lib.w4a8_midgroup_gemm(16, 16, 16, 16, Ma, Ma, 16, 16, 16, 16, 16, None, 16, 100000, 128, None)
        assert rc == 5 and b"too many groups" in lib.w4a8_last_error()
