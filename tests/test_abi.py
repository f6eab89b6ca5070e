"""CPU checks of the drop-in boundary: the library loads, exports every symbol
the headers declare (C ABI and the reference-named C++ shims), and rejects bad
arguments on the host before any GPU call (no compute is launched here)."""
import ctypes
import re
import subprocess

import pytest

import quantlib_amd as ql
from conftest import ROOT

INVALID = ql.HIP_ERROR_INVALID_VALUE

# Itanium-mangled names of the reference-named C++ shims (quantlib_compat.h).
COMPAT_MANGLED = {
    "launch_rmsnorm": "_Z14launch_rmsnormPKfS0_PfiifP12ihipStream_t",
    "launch_rope": "_Z11launch_ropePfiiifP12ihipStream_t",
    "launch_swiglu": "_Z13launch_swigluPKfS0_PfiiP12ihipStream_t",
    "launch_softmax": "_Z14launch_softmaxPKfPfiiP12ihipStream_t",
    "launch_fp16_rmsnorm": "_Z19launch_fp16_rmsnormPK6__halfS1_PS_iifP12ihipStream_t",
    "launch_fp16_rope": "_Z16launch_fp16_ropeP6__halfiiifP12ihipStream_t",
    "launch_fp16_swiglu": "_Z18launch_fp16_swigluPK6__halfS1_PS_iiP12ihipStream_t",
    "launch_fp16_embed": "_Z17launch_fp16_embedPK6__halfPS_iiP12ihipStream_t",
    "launch_fp16_add": "_Z15launch_fp16_addP6__halfPKS_iP12ihipStream_t",
    "launch_fp16_to_fp32": "_Z19launch_fp16_to_fp32PK6__halfPfiP12ihipStream_t",
    "launch_fp32_to_fp16": "_Z19launch_fp32_to_fp16PKfP6__halfiP12ihipStream_t",
    "launch_flash_attention": "_Z22launch_flash_attentionPK6__halfS1_S1_PS_iiiiiP12ihipStream_t",
    "fp16_greedy_sample": "_Z18fp16_greedy_samplePKfiP12ihipStream_t",
    "add_residual": "_Z12add_residualPfPKfiP12ihipStream_t",
    "launch_embed": "_Z12launch_embedPfPKfiiP12ihipStream_t",
    "launch_fp16_kvcache_append": "_Z26launch_fp16_kvcache_appendP6__halfS0_PKS_S2_iiiiiiP12ihipStream_t",
    "kvcache_create": "_Z14kvcache_createiiii",
    "kvcache_free": "_Z12kvcache_freeP7KVCache",
    "kvcache_append": "_Z14kvcache_appendP7KVCacheiPKfS2_P12ihipStream_t",
    "kvcache_get_k": "_Z13kvcache_get_kP7KVCachei",
    "kvcache_get_v": "_Z13kvcache_get_vP7KVCachei",
    "fp16_kvcache_create": "_Z19fp16_kvcache_createiiii",
    "fp16_kvcache_free": "_Z17fp16_kvcache_freeP11FP16KVCache",
    "paged_kv_create": "paged_kv_create",
    "paged_kv_free": "paged_kv_free",
    "paged_kv_allocate_block": "paged_kv_allocate_block",
    "paged_kv_free_block": "paged_kv_free_block",
    "quantlib_fp16_to_fp8_e4m3": "quantlib_fp16_to_fp8_e4m3",
    "quantlib_fp16_to_fp8_e5m2": "quantlib_fp16_to_fp8_e5m2",
    "quantlib_fp8_to_fp16": "quantlib_fp8_to_fp16",
    "quantlib_fp8_gemm": "quantlib_fp8_gemm",
    "quantlib_free": "quantlib_free",
    "quantlib_quant_error": "quantlib_quant_error",
    "quantlib_print_stats": "quantlib_print_stats",
}


def test_library_loads_and_reports_version():
    assert ql.version() == 100


def test_every_c_abi_symbol_declared_is_exported_and_bound():
    declared = ql.declared_symbols()
    assert len(declared) >= 20
    h = ql.lib()
    for name in declared:
        assert hasattr(h, name), name
    assert set(declared) == set(ql.SIGNATURES), set(declared) ^ set(ql.SIGNATURES)


def test_every_compat_name_is_declared_and_exported():
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "quantlib_compat.h").read_text(), flags=re.S)
    declared = set(re.findall(r"\b([a-z_0-9]+)\s*\(", text)) - {"defined"}
    assert declared == set(COMPAT_MANGLED), declared ^ set(COMPAT_MANGLED)
    out = subprocess.run(["nm", "-D", "--defined-only", str(ql.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name, mangled in COMPAT_MANGLED.items():
        assert mangled in exported, (name, mangled)


# Host-side validation: each call below must return hipErrorInvalidValue
# (or hipSuccess for an empty problem) without touching the GPU.
P = 4096  # a non-null, 16-byte aligned dummy address: never dereferenced on these paths


@pytest.mark.parametrize("call,expect", [
    (("ql_rmsnorm_f32", P, P, P, -1, 16, 1e-5, None), INVALID),
    (("ql_rmsnorm_f32", P, P, P, 4, -1, 1e-5, None), INVALID),
    (("ql_rmsnorm_f32", P, P, P, 4, 0, 1e-5, None), INVALID),
    (("ql_rmsnorm_f32", None, P, P, 4, 16, 1e-5, None), INVALID),
    (("ql_rmsnorm_f16", P, None, P, 4, 16, 1e-5, None), INVALID),
    (("ql_rmsnorm_f32", None, None, None, 0, 16, 1e-5, None), 0),
    (("ql_add_rmsnorm_f16", P, None, P, P, 4, 16, 1e-5, None), INVALID),
    (("ql_add_f32", P, P, -5, None), INVALID),
    (("ql_add_f16", None, P, 5, None), INVALID),
    (("ql_add_f16", None, None, 0, None), 0),
    (("ql_rope_f32", P, P, 4, 8, 2, 63, 504, 126, None, 0, 1e4, 0, None), INVALID),   # odd d
    (("ql_rope_f32", P, P, 4, 8, 2, 4096, 8 * 4096, 2 * 4096, None, 0, 1e4, 0, None), INVALID),  # d>2048
    (("ql_rope_f16", P, P, 4, 8, 2, 64, 100, 128, None, 0, 1e4, 0, None), INVALID),  # q stride < H*d
    (("ql_rope_f16", P, P, 4, 8, 2, 64, 512, 128, None, 0, 1e4, 2, None), INVALID),  # pairing
    (("ql_rope_f16", P, P, 4, 8, 2, 64, 512, 128, None, 0, 0.0, 0, None), INVALID),  # theta
    (("ql_rope_f16", None, None, 4, 8, 2, 64, 512, 128, None, 0, 1e4, 0, None), 0),  # nothing to do
    (("ql_swiglu_f32", P, P, P, 3, -1, None), INVALID),
    (("ql_swiglu_f16", P, None, P, 3, 8, None), INVALID),
    (("ql_swiglu_f16", None, None, None, 0, 8, None), 0),
    (("ql_softmax_f32", P, P, 2, 0, None), INVALID),
    (("ql_softmax_f16", None, P, 2, 8, None), INVALID),
    (("ql_embed_f16", P, None, 4, 100, 64, P, None), INVALID),
    (("ql_embed_f32", P, P, -1, 100, 64, P, None), INVALID),
    (("ql_embed_f16", P + 1, P, 4, 100, 64, P, None), INVALID),             # table not element-aligned
    (("ql_embed_f32", P, P, 4, 100, 64, P + 2, None), INVALID),             # out not element-aligned
    (("ql_embed_token_f16", None, 3, 64, P, None), INVALID),
    (("ql_kv_append_f32", P, P, P, P, 2, 0, 1, 8, 128, 16, 2, None), INVALID),   # layer == n_layers
    (("ql_kv_append_f32", P, P, P, P, 0, 15, 2, 8, 128, 16, 2, None), INVALID),  # pos+T > max_seq
    (("ql_kv_append_f16", P, None, P, P, 0, 0, 1, 8, 128, 16, 2, None), INVALID),
    (("ql_kv_append_f16", None, None, None, None, 0, 3, 0, 8, 128, 16, 2, None), 0),
    (("ql_paged_kv_append_f16", P, P, 4, P, P, P, 10, 4, 4, 8, 128, None), INVALID),  # layer
    (("ql_paged_kv_append_f16", P, None, 4, P, P, P, 10, 0, 4, 8, 128, None), INVALID),
    (("ql_f16_to_f32", P, P, -1, None), INVALID),
    (("ql_f32_to_f16", P, P, -1, None), INVALID),
    (("ql_f32_to_f16", P, None, 5, None), INVALID),
    (("ql_f32_to_f16", None, None, 0, None), 0),
    # fused RoPE + append: v missing, layer out of range, v stride too small, pos+T > max_seq
    (("ql_rope_paged_kv_append_f16", P, P, None, 4, 8, 2, 64, 512, 128, 128, None, 0, 1e4, 1,
      P, P, 4, P, 0, 2, None), INVALID),
    (("ql_rope_paged_kv_append_f16", P, P, P, 4, 8, 2, 64, 512, 128, 128, None, 0, 1e4, 1,
      P, P, 4, P, 2, 2, None), INVALID),
    (("ql_rope_q_paged_kv_append_f16", P, None, P, 4, 8, 2, 64, 512, 128, 128, None, 0, 1e4, 1,
      P, P, 4, P, 0, 2, None), INVALID),
    (("ql_rope_q_paged_kv_append_f16", P, P, P, 4, 8, 2, 64, 512, 128, 128, None, 0, 1e4, 1,
      P, P, 4, None, 0, 2, None), INVALID),
    (("ql_rope_kv_append_f16", P, P, P, 4, 8, 2, 64, 512, 128, 64, None, 0, 1e4, 1,
      P, P, 0, 0, 16, 2, None), INVALID),
    (("ql_rope_kv_append_f32", P, P, P, 4, 8, 2, 64, 512, 128, 128, None, 0, 1e4, 1,
      P, P, 0, 14, 16, 2, None), INVALID),
    (("ql_rope_kv_append_f32", P, P, P, 0, 8, 2, 64, 512, 128, 128, None, 0, 1e4, 1,
      P, P, 0, 3, 16, 2, None), 0),
    # attention: head_dim 96 unsupported, kv heads > heads, empty problem
    (("ql_flash_attention_f16", P, P, P, P, 4, 8, 2, 96, 1, None), INVALID),
    (("ql_flash_attention_f16", P, P, P, P, 4, 8, 2, 0, 1, None), INVALID),
    (("ql_flash_attention_f16", P, P, P, P, 4, 8, 2, 65, 1, None), INVALID),
    (("ql_flash_attention_f16", P, P, P, P, 4, 8, 2, 129, 1, None), INVALID),
    (("ql_flash_attention_f16", P, P, P, P, 4, 2, 8, 64, 1, None), INVALID),
    (("ql_flash_attention_f16", None, None, None, None, 0, 8, 2, 64, 1, None), 0),
    # q stride too small, stride not a multiple of 8, misaligned base, missing K
    (("ql_attention_f16", P, P, P, P, 1, 9, 8, 2, 64, 500, 128, 512, 1, None), INVALID),
    (("ql_attention_f16", P, P, P, P, 1, 9, 8, 2, 64, 516, 128, 512, 1, None), INVALID),
    (("ql_attention_f16", P + 2, P, P, P, 1, 9, 8, 2, 64, 512, 128, 512, 1, None), INVALID),
    (("ql_attention_f16", P, None, P, P, 1, 9, 8, 2, 64, 512, 128, 512, 1, None), INVALID),
    (("ql_attention_f16", None, None, None, None, 0, 9, 8, 2, 64, 512, 128, 512, 1, None), 0),
    # paged: layer out of range, head_dim 80, missing block tables, no sequences
    (("ql_paged_attention_f16", P, P, 512, 512, 4, 2, P, P, 2, P, 4, P, P, 8, 2, 2, 8, 2, 64, 1,
      None), INVALID),
    (("ql_paged_attention_f16", P, P, 640, 640, 4, 2, P, P, 2, P, 4, P, P, 8, 0, 2, 8, 2, 80, 1,
      None), INVALID),
    (("ql_paged_attention_f16", P, P, 512, 512, 4, 2, P, P, 2, None, 4, P, P, 8, 0, 2, 8, 2, 64, 1,
      None), INVALID),
    (("ql_paged_attention_f16", None, None, 512, 512, 0, 0, None, None, 0, None, 0, None, None, 0,
      0, 2, 8, 2, 64, 1, None), 0),
    # paged decode: workspace bytes without a pointer, head_dim 96, no sequences
    (("ql_paged_decode_attention_f16", P, P, 512, 512, 2, P, 100, P, 8, P, P, 8, 0, 1, 8, 2, 64,
      None, 4096, None), INVALID),
    (("ql_paged_decode_attention_f16", P, P, 768, 768, 2, P, 100, P, 8, P, P, 8, 0, 1, 8, 2, 96,
      None, 0, None), INVALID),
    (("ql_paged_decode_attention_f16", None, None, 512, 512, 0, None, 0, None, 0, None, None, 0, 0,
      1, 8, 2, 64, None, 0, None), 0),
    (("ql_paged_decode_workspace_size", 4, 8, 2, 64, 100, None), INVALID),
    # FP8: bad format / mode / granularity / group size; empty problems; GEMM without workspace
    (("ql_fp8_quantize", P, 4, 64, 2, 0, 0, 0, P, P, None), INVALID),
    (("ql_fp8_quantize", P, 4, 64, 0, 0, 0, 3, P, P, None), INVALID),
    (("ql_fp8_quantize", P, 4, 64, 0, 5, 0, 0, P, P, None), INVALID),
    (("ql_fp8_quantize", P, 4, 64, 0, 2, 0, 0, P, P, None), INVALID),
    (("ql_fp8_quantize", None, 0, 64, 0, 2, 128, 0, None, None, None), 0),
    (("ql_fp8_dequantize", P, None, 4, 64, 0, 2, 128, 1, P, None), INVALID),
    (("ql_fp8_dequantize", P, P, 4, 64, 0, 2, 128, 3, P, None), INVALID),      # no mode 3
    (("ql_fp8_quantize", P, 4, 64, 0, 2, 128, 2, P, P, None), INVALID),        # clean: decode only
    (("ql_fp8_scales", P, 4, 64, 0, 2, 128, 2, P, None), INVALID),
    (("ql_fp8_count_ref_special", P, 64, 2, P, None), INVALID),                 # format
    (("ql_fp8_count_ref_special", P, 64, 0, None, None), INVALID),              # no count
    (("ql_fp8_count_ref_special", P + 8, 64, 0, P, None), INVALID),             # unaligned codes
    (("ql_fp8_count_ref_special", None, 64, 0, P, None), INVALID),
    (("ql_engine_create_fp8", None, 16, 4, 64, 2, 128, P), INVALID),
    (("ql_engine_layer_fp8", None, P, 0, P, None, P, P, None), INVALID),
    (("ql_graph_begin", None), INVALID),
    (("ql_graph_end", None, P), INVALID),
    (("ql_graph_launch", None, None), INVALID),
    (("ql_graph_destroy", None), 0),
    (("ql_fp8_gemm_f16", P, P, P, 100, 64, 64, 0, 2, 128, 1, P, None, 0, None), INVALID),
    (("ql_fp8_gemm_f16", None, None, None, 0, 64, 64, 0, 2, 128, 1, None, None, 0, None), 0),
    (("ql_fp8_gemm_f16", None, None, None, 0, 64, 64, 1, 2, 128, 2, None, None, 0, None), 0),
    (("ql_fp8_gemm_f16", P, P, P, 4, 64, 64, 0, 2, 128, 3, P, None, 0, None), INVALID),
    (("ql_gemm_f16", P, P, P, -1, 4, 4, None), INVALID),
    (("ql_gemm_f16", None, None, None, 0, 4, 4, None), 0),
])
def test_argument_validation(call, expect):
    name, *args = call
    assert ql.raw(name, *args) == expect


def test_decode_workspace_size_host_query():
    size = ctypes.c_size_t(123)
    assert ql.raw("ql_paged_decode_workspace_size", 0, 32, 8, 128, 4096, ctypes.addressof(size)) == 0
    assert size.value == 0
    # one sequence, 8 KV heads: split so ~512 workgroups run; each split >= 256 keys
    assert ql.raw("ql_paged_decode_workspace_size", 1, 32, 8, 128, 8192, ctypes.addressof(size)) == 0
    assert size.value == 1 * 32 * 32 * 130 * 4
    # enough sequences to fill the GPU in one pass: no workspace
    assert ql.raw("ql_paged_decode_workspace_size", 64, 32, 8, 128, 8192, ctypes.addressof(size)) == 0
    assert size.value == 0


def test_contiguous_decode_workspace_size_host_query():
    size = ctypes.c_size_t()
    for h, hkv, d, kv, splits in ((32, 8, 128, 8192, 32), (32, 8, 128, 100, 1), (8, 2, 64, 4096, 16)):
        assert ql.raw("ql_decode_attention_workspace_size", h, hkv, d, kv, ctypes.byref(size)) == 0
        assert size.value == (0 if splits == 1 else h * splits * (d + 2) * 4), (h, hkv, d, kv, size.value)
    assert ql.raw("ql_decode_attention_workspace_size", 32, 8, 96, 100, ctypes.byref(size)) == INVALID
    # head_dims below 64 other than 64 run one pass without a workspace
    for d in (8, 32, 48, 63):
        size.value = 123
        assert ql.raw("ql_decode_attention_workspace_size", 32, 8, d, 8192, ctypes.byref(size)) == 0
        assert size.value == 0
        size.value = 123
        assert ql.raw("ql_paged_decode_workspace_size", 1, 32, 8, d, 8192, ctypes.byref(size)) == 0
        assert size.value == 0
    assert ql.raw("ql_decode_attention_f16", P, P, P, P, 10, 32, 8, 128, 8 * 128 - 8, None, 0, None) == INVALID
    assert ql.raw("ql_decode_attention_f16", P, P, P, P, 10, 32, 8, 128, 8 * 128, None, 64, None) == INVALID


def test_fp8_gemm_workspace_size_host_query():
    size = ctypes.c_size_t(123)
    q = lambda *a: ql.raw("ql_fp8_gemm_workspace_size", *a, ctypes.addressof(size))
    # more than 32 tokens: after the split partials (256-byte aligned), the token
    # rows fragment-major, K/64 chunks x 4 token tiles x 2 fragments of 1 KiB
    packed = lambda K, mt: (K // 64) * mt * 2 * 1024
    # 4096 x 14336 weights: 64 row blocks of 64 rows, four K-splits of fp32 partials
    assert q(64, 4096, 14336, 1, 0) == 0 and size.value == 4 * 64 * 4096 * 4 + packed(14336, 4)
    assert q(1, 4096, 14336, 2, 128) == 0 and size.value == 4 * 1 * 4096 * 4
    assert q(16, 6144, 4096, 0, 0) == 0 and size.value == 2 * 16 * 6144 * 4      # 96 blocks: two
    # enough row blocks (224 of 64 rows): no split; packed tokens only past 32 tokens
    assert q(1, 14336, 4096, 2, 128) == 0 and size.value == 0
    assert q(64, 14336, 4096, 0, 0) == 0 and size.value == packed(4096, 4)
    assert q(33, 14336, 4096, 0, 0) == 0 and size.value == packed(4096, 4)
    assert q(32, 14336, 4096, 0, 0) == 0 and size.value == 0
    # K too short to split (two chunks per wavefront)
    assert q(16, 1024, 512, 2, 128) == 0 and size.value == 0
    # more than 64 rows, or a shape the register path does not take: dequantized copy
    assert q(65, 512, 512, 2, 128) == 0 and size.value == 512 * 512 * 2
    assert q(16, 100, 256, 1, 0) == 0 and size.value == 100 * 256 * 2
    assert q(0, 512, 512, 2, 128) == 0 and size.value == 0
    assert q(1, 512, 512, 2, 0) == INVALID


def test_paged_slot_mapping_host_helper():
    table = (ctypes.c_int32 * 3)(4, 0, 7)
    slots = (ctypes.c_int32 * 40)()
    assert ql.raw("ql_paged_slot_mapping", ctypes.addressof(table), 3, 5, 40, ctypes.addressof(slots)) == 0
    want = [[4, 0, 7][(5 + i) // 16] * 16 + (5 + i) % 16 for i in range(40)]
    assert list(slots) == want
    # position beyond the table, or an unassigned (-1) block, is an error
    assert ql.raw("ql_paged_slot_mapping", ctypes.addressof(table), 3, 40, 10, ctypes.addressof(slots)) == INVALID
    bad = (ctypes.c_int32 * 2)(3, -1)
    assert ql.raw("ql_paged_slot_mapping", ctypes.addressof(bad), 2, 10, 10, ctypes.addressof(slots)) == INVALID


def test_dropin_caller_builds_and_links():
    """tests/dropin/caller.cpp calls the reference-named launchers, caches and
    quantlib functions through quantlib_compat.h alone and links against the
    built library: every name it uses resolves (the GPU run is in
    tests/test_gpu_compat.py)."""
    d = ROOT / "tests" / "dropin"
    subprocess.run(["make", "-B", "-C", str(d)], check=True, capture_output=True, text=True)
    undefined = subprocess.run(["nm", "-u", "-C", str(d / "caller")], check=True, capture_output=True,
                               text=True).stdout
    linked = subprocess.run(["nm", "-D", "--defined-only", "-C", str(ql.LIB_PATH)], check=True,
                            capture_output=True, text=True).stdout
    for name in ("launch_rmsnorm", "launch_rope", "launch_flash_attention", "kvcache_append",
                 "paged_kv_create", "quantlib_fp8_to_fp16", "launch_fp16_kvcache_append"):
        assert name in undefined and name in linked, name
