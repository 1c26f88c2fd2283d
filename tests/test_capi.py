"""The C ABI without a GPU: the library loads, exports every entry point that
include/orin_attn.h declares, and rejects bad arguments before queuing anything
(the reference layers return InvalidArgument for non-positive sizes,
kuiper/source/op/flash_attention.cpp:32-37)."""
import ctypes as C
import os
import re

import pytest

from orinmllm_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "orin_attn.h")
FAKE = C.c_void_p(0x1000)  # never dereferenced: every call below fails validation first


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\**\s+\**(orin_[a-z_0-9]+)\(",
                                 text, re.M)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = declared()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_host_queries():
    lib = _lib.load()
    assert lib.orin_attn_abi_version() == 1
    for code in (_lib.OK, _lib.ERR_INVALID_ARG, _lib.ERR_UNSUPPORTED, _lib.ERR_WORKSPACE,
                 _lib.ERR_LAUNCH):
        assert lib.orin_attn_status_string(code)
    assert lib.orin_attn_last_hip_error() == b""
    # one split needs no workspace; several splits need (head_size + 2) floats per split
    st = lib.orin_attn_decode_split_tokens(32, 32, 8, 4096, 0)
    assert st % 64 == 0 and 64 <= st <= 4096
    n = lib.orin_attn_decode_workspace_size(32, 32, 8, 128, 4096, 256)
    assert n == 32 * 32 * 16 * 130 * 4
    assert lib.orin_attn_decode_workspace_size(1, 8, 8, 64, 100, 128) == 0
    assert lib.orin_flash_attention_decode_workspace_size(32, 128, 4096) > 0


def test_invalid_arguments_are_rejected():
    lib = _lib.load()
    # non-positive sizes, inconsistent heads, null pointers
    assert lib.orin_flash_attention_prefill(0, 0, 32, 8, 128, 4, 0, 4096, 1024, FAKE, FAKE, FAKE,
                                            FAKE, _lib.DTYPE_FP16, None) == _lib.ERR_INVALID_ARG
    assert lib.orin_flash_attention_prefill(0, 16, 32, 8, 128, 3, 0, 4096, 1024, FAKE, FAKE, FAKE,
                                            FAKE, _lib.DTYPE_FP16, None) == _lib.ERR_INVALID_ARG
    assert lib.orin_flash_attention_prefill(4090, 16, 32, 8, 128, 4, 0, 4096, 1024, FAKE, FAKE,
                                            FAKE, FAKE, _lib.DTYPE_FP16,
                                            None) == _lib.ERR_INVALID_ARG
    assert lib.orin_flash_attention_prefill(0, 16, 32, 8, 128, 4, 0, 4096, 1024, None, FAKE, FAKE,
                                            FAKE, _lib.DTYPE_FP16, None) == _lib.ERR_INVALID_ARG
    assert lib.orin_mha_kernel(256, 12, 0, 256, 768, 1, 64, FAKE, FAKE, FAKE, FAKE, FAKE,
                               None) == _lib.ERR_INVALID_ARG  # pos must be < seq_len
    assert lib.orin_flash_attention_decode(-1, 32, 8, 128, 4, 0, 4096, 1024, FAKE, FAKE, FAKE,
                                           FAKE, _lib.DTYPE_FP16, None) == _lib.ERR_INVALID_ARG
    assert lib.orin_mha_kernel_gpu_pos(None, 12, 0, 256, 768, 1, 64, FAKE, FAKE, FAKE, FAKE, FAKE,
                                       None) == _lib.ERR_INVALID_ARG
    assert lib.orin_vision_attention_varlen(FAKE, FAKE, FAKE, FAKE, None, 4, 1024, 4096, 16, 72,
                                            0.0, _lib.DTYPE_BF16, None) == _lib.ERR_INVALID_ARG


def test_producer_arguments_are_rejected():
    """KV-cache writes and Q/K producers check sizes, layouts and alignment before any
    launch (no GPU is touched: every call here fails validation)."""
    lib = _lib.load()
    F16, INV, UNS = _lib.DTYPE_FP16, _lib.ERR_INVALID_ARG, _lib.ERR_UNSUPPORTED
    assert lib.orin_copy_to_kv_cache(FAKE, FAKE, None, 1024, 0, 64, F16, None) == INV
    assert lib.orin_copy_to_kv_cache(FAKE, FAKE, FAKE, 1024, -1, 64, F16, None) == INV
    assert lib.orin_copy_to_kv_cache(FAKE, FAKE, FAKE, 1024, 0, 64, 9, None) == UNS
    # paged write: source rows narrower than kv_heads*head_size, bad layout, misaligned head
    assert lib.orin_kv_cache_write_paged(FAKE, FAKE, 512, FAKE, FAKE, FAKE, 4, 8, 128, 16, 0, F16,
                                         None) == INV
    assert lib.orin_kv_cache_write_paged(FAKE, FAKE, 1024, FAKE, FAKE, FAKE, 4, 8, 128, 16, 3,
                                         F16, None) == INV
    assert lib.orin_kv_cache_write_paged(FAKE, FAKE, 8 * 36, FAKE, FAKE, FAKE, 4, 8, 36, 16, 0,
                                         F16, None) == UNS
    assert lib.orin_kv_cache_convert(FAKE, 1024, FAKE, FAKE, 10, 8, 128, 16, 0, 2, F16,
                                     None) == INV  # direction
    assert lib.orin_kv_cache_convert(FAKE, 1024, FAKE, None, 10, 8, 128, 16, 0, 0, F16,
                                     None) == INV
    assert lib.orin_rope_sin_cos_cache(FAKE, FAKE, 128, 0, 1e6, None) == INV
    assert lib.orin_rope_sin_cos_cache(FAKE, FAKE, 128, 64, -1.0, None) == INV
    # producer: the tokens must fit the cache; head sizes 64 / 128 / 256 only
    assert lib.orin_qk_norm_rope(FAKE, FAKE, FAKE, None, None, FAKE, FAKE, FAKE, FAKE, 0, 64, 60,
                                 None, 8, 32, 8, 128, 1e-6, F16, None) == INV
    assert lib.orin_qk_norm_rope(FAKE, FAKE, FAKE, None, None, FAKE, FAKE, FAKE, FAKE, 0, 64, 0,
                                 None, 8, 32, 8, 96, 1e-6, F16, None) == UNS
    assert lib.orin_vision_split_rope_transpose(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1024, 16, 71,
                                                _lib.DTYPE_BF16, None) == INV


def test_unsupported_shapes_are_rejected():
    lib = _lib.load()
    assert lib.orin_flash_attention_prefill(0, 16, 4, 4, 100, 1, 0, 64, 400, FAKE, FAKE, FAKE,
                                            FAKE, _lib.DTYPE_FP16,
                                            None) == _lib.ERR_UNSUPPORTED  # head 100
    assert lib.orin_flash_attention_prefill(0, 16, 4, 4, 128, 1, 0, 64, 512, FAKE, FAKE, FAKE,
                                            FAKE, 7, None) == _lib.ERR_UNSUPPORTED  # dtype
    assert lib.orin_flash_attention_decode(3, 4, 4, 72, 1, 0, 64, 288, FAKE, FAKE, FAKE, FAKE,
                                           _lib.DTYPE_FP16, None) == _lib.ERR_UNSUPPORTED
    # paged: block_size must be a power of two >= 8; split_tokens a multiple of 64
    args = (FAKE, FAKE, FAKE, FAKE, 2, 8, 2, 128, FAKE, 64)
    assert lib.orin_attn_decode_paged(*args, 4, 0, FAKE, 256, _lib.DTYPE_FP16, 0.0, 0, FAKE,
                                      1 << 20, None) == _lib.ERR_UNSUPPORTED
    assert lib.orin_attn_decode_paged(*args, 12, 0, FAKE, 256, _lib.DTYPE_FP16, 0.0, 0, FAKE,
                                      1 << 20, None) == _lib.ERR_UNSUPPORTED
    assert lib.orin_attn_decode_paged(*args, 16, 0, FAKE, 256, _lib.DTYPE_FP16, 0.0, 100, FAKE,
                                      1 << 20, None) == _lib.ERR_INVALID_ARG
    assert lib.orin_attn_decode_paged(*args, 16, 2, FAKE, 256, _lib.DTYPE_FP16, 0.0, 0, FAKE,
                                      1 << 20, None) == _lib.ERR_INVALID_ARG  # layout
    # the workspace must cover the splits
    assert lib.orin_attn_decode_paged(*args, 16, 0, FAKE, 1024, _lib.DTYPE_FP16, 0.0, 64, FAKE,
                                      16, None) == _lib.ERR_WORKSPACE


def test_missing_library_fails_loudly(tmp_path):
    saved = _lib._lib
    try:
        _lib._lib = None
        with pytest.raises(OSError, match="no CPU fallback"):
            _lib.load(str(tmp_path / "missing.so"))
    finally:
        _lib._lib = saved


def test_split_tokens_for_total():
    """A batch with a (row, kv head) per CU or more gets whole rows whatever its lengths;
    smaller near-uniform batches one round of long splits, ragged ones the automatic size;
    bad arguments 0.  Host-only (the CU count query falls back to 256 without a GPU)."""
    lib = _lib.load()
    f = lib.orin_attn_decode_split_tokens_for_total
    auto = lib.orin_attn_decode_split_tokens(32, 32, 8, 4096, 0)
    assert auto == 4096  # 32 x 8 = 256 units: whole rows
    assert f(32, 32, 8, 4096, 74949) == auto and f(32, 32, 8, 4096, 32 * 4096) == auto
    auto8 = lib.orin_attn_decode_split_tokens(8, 32, 8, 4096, 0)
    ragged = f(8, 32, 8, 4096, 8 * 2000)
    uniform = f(8, 32, 8, 4096, 8 * 4096)
    assert auto8 < 4096 and ragged == auto8
    assert uniform % 64 == 0 and uniform >= auto8
    assert f(0, 32, 8, 4096, 1) == 0 and f(32, 32, 7, 4096, 1) == 0 and f(32, 32, 8, 4096, -1) == 0
