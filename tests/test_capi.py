"""The C-ABI library loads on the CPU and exports exactly what include/oxr_verify.h declares,
with the argument lists the ctypes binding uses.  No compute call is made here."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from conftest import ROOT, pkg

HEADER = ROOT / "include" / "oxr_verify.h"

_CTYPE_OF = {
    "int": ctypes.c_int, "int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64, "float": ctypes.c_float,
    "size_t": ctypes.c_size_t, "oxr_stream_t": ctypes.c_void_p, "void": None,
}


def _declarations() -> dict[str, list[str]]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[\w\s\*]+?\b(oxr_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        args = [a.strip() for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(1)] = args
    return decls


def _ctype(arg: str):
    if "*" in arg:
        return "char_p" if arg.startswith("const char") else ctypes.c_void_p
    base = arg.replace("const ", "").split()[0]
    return _CTYPE_OF[base]


def test_header_declares_entry_points() -> None:
    decls = _declarations()
    for name in ("oxr_ngram_propose", "oxr_propose_verify_inputs", "oxr_qk_norm_rope_store", "oxr_accept"):
        assert name in decls


def test_library_exports_every_declared_symbol() -> None:
    lib = pkg("_lib")
    handle = ctypes.CDLL(str(lib.LIB_PATH))
    for name in _declarations():
        assert hasattr(handle, name), f"{name} declared in {HEADER.name} but not exported"


def test_ctypes_signatures_match_header() -> None:
    lib = pkg("_lib")
    decls = _declarations()
    assert set(lib.SIGNATURES) == set(decls)
    for name, args in decls.items():
        _, argtypes = lib.SIGNATURES[name]
        assert len(argtypes) == len(args), name
        for arg, bound in zip(args, argtypes):
            want = _ctype(arg)
            if want == "char_p":
                continue
            assert bound == want, (name, arg, bound)


def test_status_strings_and_version() -> None:
    lib = pkg("_lib").lib()
    assert lib.oxr_abi_version() == 1
    assert b"unsupported" in lib.oxr_status_string(-2)
    assert lib.oxr_status_string(0) == b"ok"


def test_entry_points_reject_bad_arguments_before_launch() -> None:
    """Validation happens on the host: invalid sizes return an error code and launch nothing."""
    lib = pkg("_lib").lib()
    assert lib.oxr_qk_norm_rope_store(None, None, None, None, None, 1e-6, None, None, None, 0, 4, 16, 8, 64,
                                      None, None, None, None) == -2  # head_dim != 128
    assert lib.oxr_ngram_propose(None, 0, None, None, 1, 9, 3, None, None, None, None) == -2  # max_n > 8
    assert lib.oxr_ngram_propose(None, 0, None, None, 0, 4, 3, None, None, None, None) == 0  # empty batch
    assert lib.oxr_packed_weight_elems(40, 256) == 48 * 256  # last tile zero-padded
    assert lib.oxr_packed_weight_elems(0, 256) == 0
    assert lib.oxr_pack_weight_bf16(16, 32, 100, 4096, None) == -2  # k not a multiple of 128
    assert lib.oxr_pack_weight_bf16(None, 32, 128, 4096, None) == -1  # no source
    assert lib.oxr_pack_weight_bf16(4096, 32, 128, 4096 + 64, None) == -1  # overlapping buffers
    # packed SiLU*mul needs the up rows to start a tile (n % 16 == 0)
    assert lib.oxr_gemm_bf16_packed(16, 128, 4, 32, 128, 40, 1, 4096, 40, 0, None) == -2
    assert lib.oxr_gemm_bf16_packed(16, 128, 4, 32, 128, 64, 0, 4096, 64, 4, None) == -1  # unknown flag
    # packed y needs a row length that is a multiple of 128, and no residual add
    assert lib.oxr_gemm_bf16_packed(16, 128, 4, 32, 128, 64, 0, 4096, 0, 2, None) == -2
    assert lib.oxr_gemm_bf16_packed(16, 128, 4, 32, 128, 128, 3, 4096, 0, 2, None) == -2
    assert lib.oxr_gemm_bf16_partial_packed(16, 0, 4, 32, 128, 64, 4096, 1, 2, None) == -1  # y flag on partials


def test_static_scratch_holds_every_attention_workspace() -> None:
    """Host-side sizing only (no GPU call): the fused attention's allocation-free entry point keeps its
    split partials in a static array that must hold the workspace of every shape the workspace entry
    point takes -- any batch, kv-head count and context bound."""
    handle = pkg("_lib").lib()
    limit = handle.oxr_static_scratch_bytes()
    worst = 0
    for kv in (1, 2, 3, 4, 8, 16, 32, 64):
        for batch in list(range(1, 130)) + [255, 256, 257, 511, 512, 4096]:
            for max_len in (16, 255, 256, 257, 1000, 4096, 16384, 1 << 20):
                worst = max(worst, handle.oxr_paged_extend_workspace_bytes(batch, kv, max_len))
    assert 0 < worst <= limit, (worst, limit)


def test_build_rejects_kernels_with_scratch() -> None:
    """The build's guard reads the compiler's resource-usage remarks and names every kernel with
    a nonzero ScratchSize."""
    build = pkg("build")
    remarks = (
        "a.hip:1:1: remark: Function Name: k_clean [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:9:1: remark: Function Name: k_spills [-Rpass-analysis=kernel-resource-usage]\n"
        "a.hip:9:1: remark:     ScratchSize [bytes/lane]: 56 [-Rpass-analysis=kernel-resource-usage]\n"
    )
    assert build.scratch_users(remarks) == [("k_spills", 56)]


def test_attention_plan_sizes_and_short_plans_refused() -> None:
    """Host side of the context-piece plans (no GPU call): a plan exists exactly when the launch
    splits its contexts (2 + B + 3 * B * splits entries, B = 8 at 16/8 heads: 8 splits), and the
    planned launches refuse a missing or shorter plan before launching anything."""
    lib = pkg("_lib").lib()
    assert lib.oxr_paged_extend_plan_ints(8, 4, 16, 8, 4112) == 2 + 8 + 3 * 8 * 8
    assert lib.oxr_paged_extend_plan_ints(512, 4, 16, 8, 4112) == 0  # 2048 units: one piece each
    assert lib.oxr_paged_extend_plan_ints(0, 4, 16, 8, 4112) == 0
    need = lib.oxr_paged_extend_plan_ints(8, 4, 16, 8, 4112)
    p = ctypes.c_void_p(16)  # never dereferenced: the checks come first
    args = (p, p, p, p, p, 257, 8, 4, 16, 8, 128, 16, 65536, 4112, 0.088, p, p, 1 << 30)
    assert lib.oxr_paged_extend_planned(*args, None, need, None) == -1
    assert lib.oxr_paged_extend_planned(*args, p, need - 1, None) == -1
    fused = (p, p, p, p, p, 4200, p, 1e-6, p, p, p, 1 << 20, p, p, 257, 8, 4, 16, 8, 128, 16, 65536, 4112, 0.088, p,
             0, p, 1 << 30)
    assert lib.oxr_qk_norm_rope_paged_extend_planned(*fused, p, need - 1, None) == -1


def test_lm_head_accept_refusals() -> None:
    """Host checks of oxr_lm_head_accept_packed (no GPU call): the token rows must be exactly
    batch * tokens_per_seq, at most 256 of them and at most 256 per sequence; acceptance arguments
    are checked as oxr_accept checks them; a batch of 0 launches nothing."""
    lib = pkg("_lib").lib()
    p = ctypes.c_void_p(16)  # never dereferenced: the checks come first

    def call(m, k, s, batch, predicted=p, draft_len=p, history=None, history_len=None):
        return lib.oxr_lm_head_accept_packed(p, m, p, 2048, 151936, p, 1 << 30, predicted, p, draft_len, k, s,
                                             batch, -1, None, p, None, None, None, history, 0, history_len, None,
                                             None)

    assert call(33, 3, 4, 8) == -1     # m != batch * tokens_per_seq
    assert call(32, 3, 4, 8, predicted=None) == -1
    assert call(32, 3, 4, 8, draft_len=None) == -1
    assert call(32, 3, 4, 8, history=p) == -1  # history without history_len
    assert call(32, -1, 4, 8) == -1
    assert call(260, 3, 4, 65) == -2   # more than 256 rows
    assert call(257, 256, 257, 1) == -2  # more than 256 rows per sequence
    assert call(0, 3, 4, 0) == 0
