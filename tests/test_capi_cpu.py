"""The C ABI on the CPU: the shared library loads, exports every symbol the public header
declares, and its host-side validation rejects bad arguments before any launch (these
calls never touch a GPU, so they run anywhere)."""
import ctypes

import pytest

from cuda_transformer_amd import capi

OK, INVALID, HEADDIM, LAYOUT = 0, 1, 2, 3


def test_library_exports_every_declared_symbol():
    lib = capi.lib()
    declared = capi.declared_symbols()
    assert len(declared) >= 20
    missing = [name for name in declared if not hasattr(lib, name)]
    assert missing == []
    assert set(declared) == set(capi.SIGNATURES), "ctypes prototypes out of sync with the header"


def test_version_and_last_error():
    lib = capi.lib()
    assert lib.cta_version().decode().startswith("cuda_transformer_amd")
    assert isinstance(lib.cta_last_error(), bytes)


def _fwd(hs=64, B=1, nh=1, T=8, q=16, s=(512, 512, 64, 1), o=16, l=16):
    st = capi.strides(s)
    return capi.lib().cta_flash_attention_fwd(q, st, q, st, q, st, B, nh, T, hs, 1, o, l, None)


def test_unsupported_head_dim_message_matches_reference():
    lib = capi.lib()
    assert _fwd(hs=48) == HEADDIM
    assert lib.cta_last_error().decode() == (
        "Unsupported head dimension! Only hs=32, hs=64, and hs=128 are supported.")


def test_empty_and_invalid_sizes():
    assert _fwd(T=0) == OK           # nothing to do, no launch
    assert _fwd(B=0) == OK
    assert _fwd(T=-1) == INVALID


def test_layout_checks_run_before_launch():
    # misaligned pointer / non-unit d-stride / stride not divisible by 4 -> CTA_ERR_LAYOUT
    assert _fwd(q=20) == LAYOUT
    assert _fwd(s=(512, 512, 64, 2)) == LAYOUT
    assert _fwd(s=(512, 512, 66, 1)) == LAYOUT
    assert b"16-byte" in capi.lib().cta_last_error()
    # a stage of 64 rows must fit 32-bit byte offsets: time strides in [0, 2^23)
    assert _fwd(s=(1 << 24, 1 << 24, 1 << 23, 1)) == LAYOUT
    assert _fwd(s=(512, 512, -64, 1)) == LAYOUT
    assert b"2^23" in capi.lib().cta_last_error()


def test_workspace_queries():
    lib = capi.lib()
    assert lib.cta_db_calculation_workspace(1, 8192, 3072) == (256 + 8) * 3072 * 4  # partials + group sums
    assert lib.cta_db_calculation_workspace(0, 5, 5) == 0
    assert lib.cta_layernorm_bwd_workspace(8192, 768) > 0
    assert lib.cta_causal_self_attention_bwd_workspace(8, 33) == 8 * 33 * 33 * 4
    assert lib.cta_cuda_fma_workspace(1, 8192, 768, 3072) == 0          # fills the GPU: no split
    assert lib.cta_cuda_fma_workspace(1, 768, 8192, 3072) > 0           # 144 tiles, K = 8192
    # weight + bias gradient: the split partials plus one row of column sums per split
    fma_ws = lib.cta_cuda_fma_workspace(1, 768, 8192, 3072)
    wb_ws = lib.cta_linear_weight_bias_grad_workspace(8192, 768, 3072)
    splits = fma_ws // (768 * 3072 * 4)
    assert splits > 1 and wb_ws == max(fma_ws + splits * 3072 * 4,
                                      lib.cta_db_calculation_workspace(1, 8192, 3072))
    assert lib.cta_linear_weight_bias_grad_workspace(0, 5, 5) == 0
    # no weight columns: db alone, still through the column-sum partials
    assert lib.cta_linear_weight_bias_grad_workspace(300, 0, 8) == lib.cta_db_calculation_workspace(1, 300, 8) > 0
    for hs in (32, 64, 128):  # 16-bit dS workspace: 2 KiB per stored 32x32 tile
        assert lib.cta_flash_attention_bwd_bf16_workspace(1, 2, 64, hs, 1) == 2 * 3 * 2048
    assert lib.cta_flash_attention_bwd_bf16_workspace(1, 2, 64, 48, 1) == 0


def test_other_entry_points_validate_arguments():
    lib = capi.lib()
    s3 = capi.strides((1, 1, 1))
    assert lib.cta_cuda_fma(16, s3, 16, s3, 16, 1, 2, 3, 4, 5, 3, 16, None, None) == INVALID  # w_batch
    # the residual LayerNorm needs its residual operand
    assert lib.cta_add_layernorm_fwd(16, None, 16, 16, 4, 8, 1e-5, 16, 16, 16, 16, None) == INVALID
    assert lib.cta_add_layernorm_fwd(16, 16, 16, 16, 4, 8, 1e-5, None, 16, 16, 16, None) == INVALID
    assert lib.cta_add_layernorm_bwd(16, 16, 16, 16, 16, None, 4, 8, 16, 16, 16, 16, None) == INVALID
    s2 = capi.strides((1, 1))
    assert lib.cta_linear_weight_bias_grad(16, s2, 16, s2, -1, 2, 3, 16, 16, None, None) == INVALID
    assert lib.cta_linear_weight_bias_grad(16, s2, 16, s2, 4, 2, 3, 16, None, None, None) == INVALID
    assert lib.cta_linear_weight_bias_grad(16, s2, 16, s2, 4, 2, 0, None, None, None, None) == OK
    # a required workspace that is missing is an error, not a launch
    assert lib.cta_linear_weight_bias_grad(None, s2, 16, s2, 300, 0, 8, None, 16, None, None) == INVALID
    assert lib.cta_linear_weight_bias_grad(16, s2, 16, s2, 300, 4, 8, 16, 16, None, None) == INVALID
    assert lib.cta_gelu_fwd(16, 16, -1, None) == INVALID
    assert lib.cta_gelu_fwd(20, 16, 8, None) == LAYOUT
    assert lib.cta_gelu_tanh_fwd(16, 16, -1, None) == INVALID
    assert lib.cta_gelu_tanh_bwd(16, 16, 20, 8, None) == LAYOUT
    assert lib.cta_gelu_tanh_bwd(16, None, 16, 8, None) == INVALID
    assert lib.cta_softmax_fwd(16, 16, -1, 4, None) == INVALID
    assert lib.cta_layernorm_fwd(16, 16, 16, 4, 0, ctypes.c_float(1e-5), 16, 16, 16, None) == INVALID
    assert lib.cta_causal_self_attention_fwd(16, 1, 4, 10, 3, 1, 16, 16, None) == INVALID  # C % nh
    with pytest.raises(capi.CtaError, match="Unsupported head dimension"):
        st = capi.strides((512, 512, 64, 1))
        capi.call("cta_flash_attention_bwd_delta", 16, st, 16, st, 1, 1, 8, 96, 16, None)


def test_half_forward_rejects_time_strides_of_2_to_24():
    # The 16-bit kernels address a stage's 64 rows with 32-bit byte offsets; larger time
    # strides are refused before any launch.
    lib = capi.lib()
    ok = capi.strides((512, 512, 64, 1))
    big = capi.strides((1 << 32, 1 << 32, 1 << 31, 1))
    args = (1, 1, 8, 64, 1, 16, 16, None)
    assert lib.cta_flash_attention_fwd_bf16(16, big, 16, ok, 16, ok, *args) == LAYOUT
    assert b"2^24" in lib.cta_last_error()
    edge = capi.strides((1 << 24, 1 << 24, 1 << 24, 1))  # a stage's 64 rows need 32-bit offsets
    assert lib.cta_flash_attention_fwd_bf16(16, ok, 16, edge, 16, ok, *args) == LAYOUT
    assert lib.cta_flash_attention_fwd_f16(16, ok, 16, ok, 16, big, *args) == LAYOUT


def test_header_is_plain_c_and_links(tmp_path):
    # A C caller (the cgo / FFI case): the header compiles as strict C99, the library links
    # from C, and an argument error comes back as a status code and a message.
    import shutil
    import subprocess
    from pathlib import Path

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    repo = Path(__file__).resolve().parents[1]
    lib_dir = repo / "cuda_transformer_amd"
    src = tmp_path / "caller.c"
    src.write_text(
        '#include <stdio.h>\n#include "cuda_transformer_amd.h"\n'
        "int main(void) {\n"
        "  const int64_t s[4] = {512, 512, 64, 1};\n"
        "  int rc = cta_flash_attention_fwd((const float*)16, s, (const float*)16, s,\n"
        "                                   (const float*)16, s, 1, 1, 8, 64, 1, 0, 0, 0);\n"
        '  printf("%d %s\\n", rc, cta_last_error());\n'
        "  return rc == CTA_ERR_INVALID_ARGUMENT ? 0 : 1;\n"
        "}\n")
    exe = tmp_path / "caller"
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror",
                    f"-I{repo / 'include'}", str(src), f"-L{lib_dir}", "-lcuda_transformer_amd",
                    f"-Wl,-rpath,{lib_dir}", "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "null output pointer" in out.stdout
