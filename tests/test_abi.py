"""The C ABI boundary on the CPU: the library loads, exports exactly what
include/nspeech_rocm.h declares, validates arguments before touching the GPU,
and fails loudly (no CPU fallback) when there is no GPU."""
import ctypes as C
import re
import subprocess

import pytest
import torch

from nspeech_amd import abi

NULL = None


def test_library_exports_every_declared_function():
    L = abi.lib()
    declared = abi.header_functions()
    assert len(declared) >= 13
    for name in declared:
        assert hasattr(L, name), f"{name} declared in include/nspeech_rocm.h but not exported"
    out = subprocess.run(["nm", "-D", "--defined-only", str(abi.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (nsr_[a-z0-9_]+)$", out, flags=re.M))
    assert exported == set(declared), exported ^ set(declared)


def test_embedded_code_objects_are_gfx950():
    out = subprocess.run(["nm", "-D", "--defined-only", str(abi.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    units = re.findall(r" R nsr_co_([a-z0-9_]+)$", out, flags=re.M)
    from nspeech_amd import build

    assert sorted(units) == sorted(build.UNITS)
    for u in units:
        p = abi.LIB_DIR / f"nsr_{u}_gfx950.hsaco"
        head = p.read_bytes()[:64]
        assert head[:4] == b"\x7fELF" and head[18] == 0xE0  # EM_AMDGPU
        assert b"gfx950" in p.read_bytes()


def test_version_and_header_is_plain_c():
    assert "gfx950" in abi.version()
    text = abi.HEADER.read_text()
    assert "torch" not in text and "hip_runtime" not in text


@pytest.mark.parametrize("call", [
    lambda L: L.nsr_layernorm(NULL, 0, NULL, NULL, 0, 16, 0, 4, 8, 8, 8, C.c_float(1e-5), 0, 0, NULL),
    lambda L: L.nsr_layernorm(16, 0, NULL, NULL, 0, 16, 0, 4, 0, 8, 8, C.c_float(1e-5), 0, 0, NULL),
    lambda L: L.nsr_layernorm(16, 0, NULL, NULL, 0, 16, 0, 4, 8, 4, 8, C.c_float(1e-5), 0, 0, NULL),
    lambda L: L.nsr_layernorm(16, 7, NULL, NULL, 0, 16, 0, 4, 8, 8, 8, C.c_float(1e-5), 0, 0, NULL),
    lambda L: L.nsr_layernorm(16, 0, NULL, NULL, 2, 16, 0, 4, 8, 8, 8, C.c_float(1e-5), 0, 0, NULL),
    lambda L: L.nsr_layernorm(16, 0, NULL, NULL, 0, 16, 0, 4, 8, 8, 8, C.c_float(1e-5), 4, 0, NULL),
    lambda L: L.nsr_layernorm(16, 0, NULL, NULL, 0, 16, 0, 4, 8, 8, 8, C.c_float(1e-5), 0, 9, NULL),
    lambda L: L.nsr_residual_add_layernorm(16, 0, NULL, 0, NULL, 0, NULL, NULL, 0, 16, 0, 4, 8, C.c_float(1e-5),
                                           0, 0, NULL),
    lambda L: L.nsr_rope_table_f32(NULL, 4, 32, C.c_float(1e4)),
    lambda L: L.nsr_rope_table_f32(16, 4, 31, C.c_float(1e4)),
    lambda L: L.nsr_rotary_partial_interleaved_f32(16, 16, 16, 16, 1, 8, 8, 16, 64, 34, C.c_float(1e4), 0, NULL, 0,
                                                   NULL),
    lambda L: L.nsr_rotary_partial_interleaved_f32(16, 16, 16, 16, 1, 8, 8, 16, 64, 66, C.c_float(1e4), 0, NULL, 0,
                                                   NULL),
    lambda L: L.nsr_rotary_partial_interleaved_f32(16, 16, 16, NULL, 1, 8, 8, 16, 64, 32, C.c_float(1e4), 0, NULL,
                                                   0, NULL),
    lambda L: L.nsr_rotary_partial_interleaved_f32(17, NULL, 16, NULL, 1, 8, 8, 16, 64, 32, C.c_float(1e4), 0,
                                                   NULL, 0, NULL),
    lambda L: L.nsr_rotary_partial_interleaved_f32(16, NULL, 16, NULL, 1, 8, 8, 16, 64, 32, C.c_float(1e4), 8, 16,
                                                   20, NULL),
    lambda L: L.nsr_adain_snake_f32(16, 16, 16, 16, 0, 0, 0, 16, 1, 4, 0, C.c_float(1e-5), NULL),
    lambda L: L.nsr_adain_snake_f32(16, NULL, 16, 16, 0, 0, 0, 16, 1, 4, 100, C.c_float(1e-5), NULL),
    lambda L: L.nsr_adain_snake_f32(16, 16, 16, 16, 2, 0, 0, 16, 1, 4, 100, C.c_float(1e-5), NULL),
    # f16 AdaIN+Snake: null gamma, odd address, out at another offset within 16 bytes than x, row too long
    lambda L: L.nsr_adain_snake_f16(16, NULL, 16, 16, 0, 0, 0, 16, 1, 4, 100, C.c_float(1e-5), NULL),
    lambda L: L.nsr_adain_snake_f16(17, 16, 16, 16, 0, 0, 0, 17, 1, 4, 100, C.c_float(1e-5), NULL),
    lambda L: L.nsr_adain_snake_f16(16, 16, 16, 16, 0, 0, 0, 18, 1, 4, 100, C.c_float(1e-5), NULL),
    lambda L: L.nsr_adain_snake_f16(16, 16, 16, 16, 0, 0, 0, 16, 1, 4, 131073, C.c_float(1e-5), NULL),
    lambda L: L.nsr_q8_0_embed_gather(16, 100, 48, 16, 0, 4, 16, 0, NULL, NULL),
    lambda L: L.nsr_q8_0_embed_gather(16, 100, 64, 16, 0, 4, 20, 0, NULL, NULL),
    lambda L: L.nsr_q8_0_embed_gather(17, 100, 64, 16, 0, 4, 16, 0, NULL, NULL),
    lambda L: L.nsr_q8_0_embed_gather(16, 0, 64, 16, 0, 4, 16, 0, NULL, NULL),
    lambda L: L.nsr_activation(16, 16, 0, 100, 0, NULL),
    lambda L: L.nsr_activation(16, 16, 5, 100, 1, NULL),
    lambda L: L.nsr_glu_silu(NULL, 16, 0, 100, NULL),
    lambda L: L.nsr_residual_add(16, NULL, 16, 0, 100, NULL),
    # decode RoPE + cache: odd head_dim, rotary_dim > head_dim, pos outside the cache, bf16, v without cache_v,
    # misaligned f16 q, table too short
    lambda L: L.nsr_rope_qk_cache_append(16, 16, NULL, 1, 16, 8, 16, NULL, 2, 2, 63, 32, 0, 8, NULL),
    lambda L: L.nsr_rope_qk_cache_append(16, 16, NULL, 1, 16, 8, 16, NULL, 2, 2, 64, 66, 0, 8, NULL),
    lambda L: L.nsr_rope_qk_cache_append(16, 16, NULL, 1, 16, 8, 16, NULL, 2, 2, 64, 32, 8, 8, NULL),
    lambda L: L.nsr_rope_qk_cache_append(16, 16, NULL, 2, 16, 8, 16, NULL, 2, 2, 64, 32, 0, 8, NULL),
    lambda L: L.nsr_rope_qk_cache_append(16, 16, 16, 1, 16, 8, 16, NULL, 2, 2, 64, 32, 0, 8, NULL),
    lambda L: L.nsr_rope_qk_cache_append(18, 16, NULL, 1, 16, 8, 16, NULL, 2, 2, 64, 32, 0, 8, NULL),
    lambda L: L.nsr_rope_qk_cache_append(16, 16, NULL, 1, 16, 3, 16, NULL, 2, 2, 64, 32, 5, 8, NULL),
    lambda L: L.nsr_kv_cache_append(NULL, 16, 1, 2, 64, 8, 0, NULL),
    lambda L: L.nsr_kv_cache_append(16, 16, 1, 2, 64, 8, -1, NULL),
    # Q8 GEMV: K not a multiple of 32, N not a multiple of 16, misaligned qs, bf16 output, null x, K == 0,
    # GLU with misaligned scales, resadd_ln without residual, bf16 LN weight
    lambda L: L.nsr_gemv_q8(16, 1, 16, 16, NULL, 16, 1, 40, 64, NULL),
    lambda L: L.nsr_gemv_q8(16, 1, 16, 16, NULL, 16, 1, 64, 40, NULL),
    lambda L: L.nsr_gemv_q8(16, 1, 24, 16, NULL, 16, 1, 64, 64, NULL),
    lambda L: L.nsr_gemv_q8(16, 1, 16, 16, NULL, 16, 2, 64, 64, NULL),
    lambda L: L.nsr_gemv_q8(NULL, 1, 16, 16, NULL, 16, 1, 64, 64, NULL),
    lambda L: L.nsr_gemv_q8(16, 1, 16, 16, NULL, 16, 1, 0, 64, NULL),
    lambda L: L.nsr_gemv_q8_bias_glu(16, 1, 16, 40, 16, 16, 1, 64, 64, NULL),
    lambda L: L.nsr_gemv_q8_resadd_ln(16, 1, 16, 16, NULL, 16, 16, 1, 16, 1, 64, 64, C.c_float(1e-5), NULL),
    lambda L: L.nsr_gemv_q8_resadd_ln(16, 1, 16, 16, 16, 16, 16, 2, 16, 1, 64, 64, C.c_float(1e-5), NULL),
    # t4 packing: K not a multiple of 32, GLU with NW not a multiple of 32, misaligned output; t4 GEMV with x
    # not aligned to 4 elements
    lambda L: L.nsr_q8_pack_t4(16, 16, 40, 64, 0, 16, 16, NULL),
    lambda L: L.nsr_q8_pack_t4(16, 16, 64, 48, 1, 16, 16, NULL),
    lambda L: L.nsr_q8_pack_t4(16, 16, 64, 64, 0, 24, 16, NULL),
    lambda L: L.nsr_gemv_q8_t4(18, 1, 16, 16, NULL, 16, 1, 64, 64, NULL),
    lambda L: L.nsr_gemv_q8_t4_bias_glu(16, 1, 16, 16, NULL, 16, 1, 64, 40, NULL),
    lambda L: L.nsr_gemv_q8_t4_resadd_ln(16, 1, 16, 16, NULL, 16, 16, 1, 16, 1, 64, 64, C.c_float(1e-5), NULL),
    # GGUF Q8_0 -> GEMV layouts: N not a multiple of 16, GLU with N not a multiple of 32, odd blocks pointer,
    # K not a multiple of 32
    lambda L: L.nsr_q8_0_to_gemv_q8(16, 40, 64, 16, 16, NULL),
    lambda L: L.nsr_q8_0_to_t4(16, 48, 64, 1, 16, 16, NULL),
    lambda L: L.nsr_q8_0_to_gemv_q8(17, 64, 64, 16, 16, NULL),
    lambda L: L.nsr_q8_0_to_t4(16, 64, 48, 0, 16, 16, NULL),
    # decode attention: head_dim not a multiple of 4, head_dim > 128, kv_len 0, more KV heads than query heads,
    # misaligned K, stride_kv_seq < head_dim, no partial buffer, no splits, null q
    lambda L: L.nsr_attention_splitkv_f16(16, 16, 16, 16, 16, 8, 6, 2, 4, C.c_float(0.125), 64, 8, 2, NULL),
    lambda L: L.nsr_attention_splitkv_f16(16, 16, 16, 16, 16, 8, 132, 2, 4, C.c_float(0.125), 1056, 132, 2, NULL),
    lambda L: L.nsr_attention_splitkv_f16(16, 16, 16, 16, 16, 0, 64, 2, 4, C.c_float(0.125), 512, 64, 2, NULL),
    lambda L: L.nsr_attention_splitkv_f16(16, 16, 16, 16, 16, 8, 64, 8, 4, C.c_float(0.125), 512, 64, 2, NULL),
    lambda L: L.nsr_attention_splitkv_f16(16, 18, 16, 16, 16, 8, 64, 2, 4, C.c_float(0.125), 512, 64, 2, NULL),
    lambda L: L.nsr_attention_splitkv_f16(16, 16, 16, 16, 16, 8, 64, 2, 4, C.c_float(0.125), 512, 32, 2, NULL),
    lambda L: L.nsr_attention_splitkv_f16(16, 16, 16, 16, NULL, 8, 64, 2, 4, C.c_float(0.125), 512, 64, 2, NULL),
    lambda L: L.nsr_attention_splitkv_f16(16, 16, 16, 16, 16, 8, 64, 2, 4, C.c_float(0.125), 512, 64, 0, NULL),
    lambda L: L.nsr_attention_decode_f16(NULL, 16, 16, 16, 8, 64, 2, 4, C.c_float(0.125), 512, 64, NULL),
    # Kokoro tail: null input, negative n, misaligned pointer; iSTFT out_len past (n_frames - 1) * hop,
    # hop not dividing n_fft, an n_fft with no kernel, no frames, null output
    lambda L: L.nsr_resblock_average_f32(16, NULL, 16, 16, 8, 0, C.c_float(0.0), NULL),
    lambda L: L.nsr_scale_f32(16, 16, -1, C.c_float(2.0), NULL),
    lambda L: L.nsr_leaky_relu_f32(18, 16, 8, C.c_float(0.01), NULL),
    lambda L: L.nsr_istft_f32(16, 16, 10, 46, 20, 5, NULL),
    lambda L: L.nsr_istft_f32(16, 16, 10, 20, 20, 3, NULL),
    lambda L: L.nsr_istft_f32(16, 16, 10, 20, 24, 4, NULL),
    lambda L: L.nsr_istft_f32(16, 16, 0, 0, 20, 5, NULL),
    lambda L: L.nsr_istft_f32(16, NULL, 10, 20, 20, 5, NULL),
    # chained conv: null out_stats for the plain conv, misaligned statistics, C_in not a multiple of 16
    lambda L: L.nsr_conv1d_f16w_packed_stats(16, 16, NULL, NULL, 16, NULL, 1, 16, 16, 64, 3, 1, 1,
                                             C.c_float(1e-5), 256, 1 << 20, NULL),
    lambda L: L.nsr_adain_snake_conv1d_chain_f32(16, 20, 16, 16, 16, 0, 0, 0, 16, NULL, NULL, 16, NULL, 1, 16, 16,
                                                 64, 3, 1, 1, C.c_float(1e-5), 256, 1 << 20, NULL),
    lambda L: L.nsr_adain_snake_conv1d_chain_f32(16, NULL, 16, 16, 16, 0, 0, 0, 16, NULL, NULL, 16, 20, 1, 16, 16,
                                                 64, 3, 1, 1, C.c_float(1e-5), 256, 1 << 20, NULL),
    lambda L: L.nsr_conv1d_f16w_packed_stats(16, 16, NULL, NULL, 16, 16, 1, 24, 16, 64, 3, 1, 1,
                                             C.c_float(1e-5), 256, 1 << 20, NULL),
    # conv workspaces: missing, too small, misaligned (256 bytes needed); unknown part flags
    lambda L: L.nsr_conv1d_f16w_packed_stats(16, 16, NULL, NULL, 16, 16, 1, 16, 16, 64, 3, 1, 1,
                                             C.c_float(1e-5), NULL, 0, NULL),
    lambda L: L.nsr_conv1d_f16w_packed_stats(16, 16, NULL, NULL, 16, 16, 1, 16, 16, 64, 3, 1, 1,
                                             C.c_float(1e-5), 256, 16, NULL),
    lambda L: L.nsr_conv1d_f32io(16, 16, NULL, 16, 1, 16, 16, 64, 3, 1, 1, 1, 272, 1 << 20, NULL),
    lambda L: L.nsr_adain_snake_conv1d_f32(16, 16, 16, 16, 0, 0, 0, 16, NULL, NULL, 16, 1, 16, 16, 64, 3, 1, 1,
                                           C.c_float(1e-5), NULL, 0, NULL),
    lambda L: L.nsr_conv1d_workspace_bytes(1, 16, 16, 64, 3, 1, 1, 16, C.byref(C.c_int64())),
    # snake: bf16 x, seq_len not dividing n_elements, zero channels, misaligned f32 x
    lambda L: L.nsr_snake(16, 2, 16, 0, 16, 8, 1, 8, NULL),
    lambda L: L.nsr_snake(16, 0, 16, 0, 16, 10, 1, 4, NULL),
    lambda L: L.nsr_snake(16, 0, 16, 0, 16, 8, 0, 8, NULL),
    lambda L: L.nsr_snake(18, 0, 16, 0, 16, 8, 1, 8, NULL),
])
def test_invalid_arguments_are_rejected_before_any_launch(call):
    L = abi.lib()
    st = call(L)
    assert st in (abi.NSR_ERR_BAD_ARG, abi.NSR_ERR_UNSUPPORTED), st
    assert L.nsr_last_error().decode()


def test_empty_inputs_are_no_ops():
    L = abi.lib()
    assert L.nsr_layernorm(16, 0, NULL, NULL, 0, 16, 0, 0, 8, 8, 8, C.c_float(1e-5), 0, 0, NULL) == abi.NSR_OK
    assert L.nsr_q8_0_embed_gather(16, 100, 64, 16, 0, 0, 16, 0, NULL, NULL) == abi.NSR_OK
    assert L.nsr_activation(16, 16, 0, 0, 1, NULL) == abi.NSR_OK
    assert L.nsr_kv_cache_append(16, 16, 1, 0, 64, 8, 0, NULL) == abi.NSR_OK
    assert L.nsr_gemv_q8(16, 1, 16, 16, NULL, 16, 1, 64, 0, NULL) == abi.NSR_OK


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_no_gpu_fails_loudly():
    with pytest.raises(abi.NsrError) as ei:
        abi.init()
    assert ei.value.status in (abi.NSR_ERR_HIP, abi.NSR_ERR_NOT_INIT)
    assert abi.lib().nsr_kernel_count() == 0


def test_conv_rows_past_a_buffer_descriptor_are_unsupported():
    """Each batch's conv input / output rows are addressed through one buffer
    descriptor (a 32-bit byte range). Shapes whose per-batch rows reach 4 GiB
    are rejected before any launch; the largest shape below the limit passes
    validation (B = 0 then returns at once, with no GPU work)."""
    L = abi.lib()
    big_t = (1 << 23) - 1  # 4 * 128 * big_t = 2^32 - 512 bytes per batch
    packed = lambda B, ci, co, t: L.nsr_conv1d_f16w_packed(256, 256, NULL, NULL, 256, B, ci, co, t, 1, 0, 1,  # noqa
                                                           NULL)
    assert packed(0, 128, 128, big_t) == abi.NSR_OK
    assert packed(0, 256, 16, 1 << 22) == abi.NSR_ERR_UNSUPPORTED      # input rows: 4 * 256 * 2^22 = 2^32
    assert "buffer descriptor" in L.nsr_last_error().decode()
    assert packed(0, 16, 1024, 1 << 20) == abi.NSR_ERR_UNSUPPORTED     # output rows: 4 * 1024 * 2^20 = 2^32
    assert packed(0, 16, 1023, 1 << 20) == abi.NSR_OK
