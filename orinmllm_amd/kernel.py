"""Host mirror of OrinMLLM's ``namespace kernel`` attention entry points.

Every function keeps the name and argument order of the reference function it
replaces (paths relative to the OrinMLLM source tree) and calls the HIP library
through the C ABI.  ``tensor::Tensor`` arguments are torch tensors on the GPU
(PyTorch only provides device memory and the stream here); ``CudaConfig*`` is a
:class:`CudaConfig` carrying the stream.  The element type comes from the tensors.

Errors raise :class:`orinmllm_amd._lib.OrinAttnError`; nothing falls back to a CPU
implementation.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib


class DeviceType(enum.IntEnum):
    """base::DeviceType (kuiper/include/base/base.h:50-54)."""
    kDeviceUnknown = 0
    kDeviceCPU = 1
    kDeviceCUDA = 2


class DataType(enum.IntEnum):
    """base::DataType (kuiper/include/base/base.h:58-64) plus bf16."""
    kDataTypeUnknown = 0
    kDataTypeFp32 = 1
    kDataTypeInt8 = 2
    kDataTypeInt32 = 3
    kDataTypeFp16 = 4
    kDataTypeBf16 = 5


class AttentionType(enum.IntEnum):
    """base::AttentionType (kuiper/include/base/base.h:113-118)."""
    kAttentionMHA = 0
    kAttentionFlash1 = 1
    kAttentionFlash2 = 2


_TORCH_DTYPE = {
    torch.float32: _lib.DTYPE_FP32,
    torch.float16: _lib.DTYPE_FP16,
    torch.bfloat16: _lib.DTYPE_BF16,
}


@dataclass
class CudaConfig:
    """kernel::CudaConfig (kuiper/include/base/cuda_config.h:17-33): the stream the
    kernels are queued on.  None = torch's current stream."""
    stream: Optional[torch.cuda.Stream] = None


def _stream(config: Optional[CudaConfig]) -> int:
    s = config.stream if config is not None and config.stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _ptr(t: Optional[torch.Tensor], name: str) -> Optional[int]:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the attention kernels have no CPU path)")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def _dtype(*ts: torch.Tensor) -> int:
    dt = ts[0].dtype
    for t in ts[1:]:
        if t.dtype != dt:
            raise ValueError(f"mixed dtypes {dt} and {t.dtype}")
    if dt not in _TORCH_DTYPE:
        raise ValueError(f"unsupported dtype {dt}")
    return _TORCH_DTYPE[dt]


def _i32(t: torch.Tensor, name: str) -> int:
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32")
    return _ptr(t, name)


# ---------------------------------------------------------------- fp32 MHA

def mha_kernel_cu(pos, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size, mha_out,
                  query_tensor, score_tensor, key_cache_tensor, value_cache_tensor,
                  device_type=DeviceType.kDeviceCUDA, config=None):
    """kernel::mha_kernel_cu (kuiper/source/op/kernels/cuda/mha_kernel.cuh:4-8)."""
    if _dtype(mha_out, query_tensor, key_cache_tensor, value_cache_tensor) != _lib.DTYPE_FP32:
        raise ValueError("mha_kernel_cu is fp32")
    _lib.check("orin_mha_kernel", _lib.load().orin_mha_kernel(
        pos, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size,
        _ptr(mha_out, "mha_out"), _ptr(query_tensor, "query"), _ptr(score_tensor, "score"),
        _ptr(key_cache_tensor, "key_cache"), _ptr(value_cache_tensor, "value_cache"),
        _stream(config)))


def mha_kernel_cu_gpu_pos(pos_ptr, head_num, layer_index, seq_len, kv_dim, kv_mul, head_size,
                          mha_out, query_tensor, score_tensor, key_cache_tensor,
                          value_cache_tensor, device_type=DeviceType.kDeviceCUDA, config=None):
    """kernel::mha_kernel_cu_gpu_pos (mha_kernel.cuh:13-19); pos_ptr: int32 GPU tensor [1]."""
    _lib.check("orin_mha_kernel_gpu_pos", _lib.load().orin_mha_kernel_gpu_pos(
        _i32(pos_ptr, "pos_ptr"), head_num, layer_index, seq_len, kv_dim, kv_mul, head_size,
        _ptr(mha_out, "mha_out"), _ptr(query_tensor, "query"), _ptr(score_tensor, "score"),
        _ptr(key_cache_tensor, "key_cache"), _ptr(value_cache_tensor, "value_cache"),
        _stream(config)))


def batched_mha_kernel_cu(start_pos, seq_len, head_num, layer_index, max_seq_len, dim, kv_dim,
                          kv_mul, head_size, mha_out, query_tensor, score_tensor,
                          key_cache_tensor, value_cache_tensor,
                          device_type=DeviceType.kDeviceCUDA, config=None):
    """kernel::batched_mha_kernel_cu (mha_kernel.cuh:21-26)."""
    _lib.check("orin_batched_mha", _lib.load().orin_batched_mha(
        start_pos, seq_len, head_num, layer_index, max_seq_len, dim, kv_dim, kv_mul, head_size,
        _ptr(mha_out, "mha_out"), _ptr(query_tensor, "query"), _ptr(score_tensor, "score"),
        _ptr(key_cache_tensor, "key_cache"), _ptr(value_cache_tensor, "value_cache"),
        _stream(config)))


def get_mha_kernel(device_type):
    """kernel::get_mha_kernel (kuiper/source/op/kernels/kernels_interfaces.cpp:63-72).

    Only the GPU kernel is provided: the reference's CPU kernel is not part of this
    library (it is restated under oracle/ as a test checker only)."""
    if DeviceType(device_type) == DeviceType.kDeviceCUDA:
        return mha_kernel_cu
    raise NotImplementedError(f"no MHA kernel for {DeviceType(device_type).name} in this library")


# ---------------------------------------------------------------- flash attention

def _prefill(start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul, layer_index,
             max_seq_len, kv_dim, query, output, key_cache, value_cache, config):
    dt = _dtype(query, output, key_cache, value_cache)
    _lib.check("orin_flash_attention_prefill", _lib.load().orin_flash_attention_prefill(
        start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul, layer_index, max_seq_len,
        kv_dim, _ptr(query, "query"), _ptr(output, "output"), _ptr(key_cache, "key_cache"),
        _ptr(value_cache, "value_cache"), dt, _stream(config)))


def flash_attention_prefill_cu(start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul,
                               layer_index, max_seq_len, kv_dim, query, output, key_cache,
                               value_cache, config=None):
    """kernel::flash_attention_prefill_cu (flash_attention_kernel.cuh:27-42) and its fp16 /
    FlashAttention-2 siblings: the element type is taken from the tensors."""
    _prefill(start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul, layer_index,
             max_seq_len, kv_dim, query, output, key_cache, value_cache, config)


flash_attention_prefill_fp16_cu = flash_attention_prefill_cu
flash_attention2_prefill_cu = flash_attention_prefill_cu
flash_attention2_prefill_fp16_cu = flash_attention_prefill_cu


def flash_attention_prefill_qk_norm_rope_cu(start_pos, seq_len, head_num, kv_head_num,
                                            head_size, kv_mul, layer_index, max_seq_len, kv_dim,
                                            query, output, key_cache, value_cache,
                                            q_norm_weight, sin_cache, cos_cache, eps=1e-6,
                                            config=None):
    """Causal prefill whose query rows are RMS-normalised (q_norm_weight, may be None) and
    rotated (sin/cos caches) as they are loaded; equals qk_norm_rope_cu on the query then
    flash_attention_prefill_cu, bit for bit.  query is left unchanged."""
    dt = _dtype(query, output, key_cache, value_cache,
                *[w for w in (q_norm_weight,) if w is not None])
    if sin_cache.dtype != torch.float32 or cos_cache.dtype != torch.float32:
        raise ValueError("sin/cos caches are fp32")
    _lib.check("orin_flash_attention_prefill_qk_norm_rope",
               _lib.load().orin_flash_attention_prefill_qk_norm_rope(
                   start_pos, seq_len, head_num, kv_head_num, head_size, kv_mul, layer_index,
                   max_seq_len, kv_dim, _ptr(query, "query"), _ptr(output, "output"),
                   _ptr(key_cache, "key_cache"), _ptr(value_cache, "value_cache"),
                   _ptr(q_norm_weight, "q_norm_weight"), _ptr(sin_cache, "sin_cache"),
                   _ptr(cos_cache, "cos_cache"), float(eps), dt, _stream(config)))


def flash_attention_decode_cu(pos, head_num, kv_head_num, head_size, kv_mul, layer_index,
                              max_seq_len, kv_dim, query, output, key_cache, value_cache,
                              config=None):
    """kernel::flash_attention_decode_cu (flash_attention_kernel.cuh:50-63) and its fp16 /
    FlashAttention-2 siblings."""
    dt = _dtype(query, output, key_cache, value_cache)
    _lib.check("orin_flash_attention_decode", _lib.load().orin_flash_attention_decode(
        pos, head_num, kv_head_num, head_size, kv_mul, layer_index, max_seq_len, kv_dim,
        _ptr(query, "query"), _ptr(output, "output"), _ptr(key_cache, "key_cache"),
        _ptr(value_cache, "value_cache"), dt, _stream(config)))


flash_attention_decode_fp16_cu = flash_attention_decode_cu
flash_attention2_decode_cu = flash_attention_decode_cu
flash_attention2_decode_fp16_cu = flash_attention_decode_cu


def flash_attention_decode_fp16_gpu_pos_cu(pos_ptr, head_num, kv_head_num, head_size, kv_mul,
                                           layer_index, max_seq_len, kv_dim, query, output,
                                           key_cache, value_cache, config=None):
    """kernel::flash_attention_decode_fp16_gpu_pos_cu (flash_attention_kernel.cuh:103-117)."""
    dt = _dtype(query, output, key_cache, value_cache)
    _lib.check("orin_flash_attention_decode_gpu_pos",
               _lib.load().orin_flash_attention_decode_gpu_pos(
                   _i32(pos_ptr, "pos_ptr"), head_num, kv_head_num, head_size, kv_mul,
                   layer_index, max_seq_len, kv_dim, _ptr(query, "query"),
                   _ptr(output, "output"), _ptr(key_cache, "key_cache"),
                   _ptr(value_cache, "value_cache"), dt, _stream(config)))


flash_attention2_decode_fp16_gpu_pos_cu = flash_attention_decode_fp16_gpu_pos_cu


def reserve_decode_workspace(head_num, head_size, max_seq_len, stream=None, prefill_bytes=0):
    """Allocate the library-owned flash-decode workspace of `stream` (a torch.cuda.Stream;
    None = the current stream) now, before that stream captures a graph."""
    lib = _lib.load()
    n = lib.orin_flash_attention_decode_workspace_size(head_num, head_size, max_seq_len)
    s = (stream if stream is not None else torch.cuda.current_stream()).cuda_stream
    _lib.check("orin_attn_workspace_reserve_stream",
               lib.orin_attn_workspace_reserve_stream(n, prefill_bytes, s))


def release_workspace(stream=None, all_streams=False):
    """Free the library-owned buffers of `stream` (a torch.cuda.Stream; None = the current
    stream), or of every stream of the current device with all_streams, after synchronising
    what may still use them; call it before destroying a stream that ran these kernels.
    Raises while one of those streams is being captured."""
    lib = _lib.load()
    if all_streams:
        _lib.check("orin_attn_workspace_release", lib.orin_attn_workspace_release())
        return
    s = (stream if stream is not None else torch.cuda.current_stream()).cuda_stream
    _lib.check("orin_attn_workspace_release_stream", lib.orin_attn_workspace_release_stream(s))


def prefill_workspace_size(start_pos, seq_len, head_num, kv_head_num, head_size, dtype):
    """Bytes of the library-owned key-split workspace one causal prefill launch needs."""
    return int(_lib.load().orin_flash_attention_prefill_workspace_size(
        start_pos, seq_len, head_num, kv_head_num, head_size, dtype))


# ---------------------------------------------------------------- batched / paged decode

def decode_workspace_size(batch, head_num, kv_head_num, head_size, max_context_len,
                          split_tokens=0):
    return int(_lib.load().orin_attn_decode_workspace_size(
        batch, head_num, kv_head_num, head_size, max_context_len, split_tokens))


def decode_split_tokens_for_total(batch, head_num, kv_head_num, max_context_len,
                                  sum_context_len):
    """Split size (pass it as split_tokens) for a batched decode whose total KV length the
    caller knows on the host; the automatic choice unless the rows are near-uniform."""
    st = int(_lib.load().orin_attn_decode_split_tokens_for_total(
        batch, head_num, kv_head_num, max_context_len, int(sum_context_len)))
    if st <= 0:
        raise _lib.OrinAttnError("orin_attn_decode_split_tokens_for_total", _lib.ERR_INVALID_ARG)
    return st


def _workspace(nbytes, workspace, device):
    if nbytes == 0:
        return None, 0
    if workspace is None:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=device)
    if workspace.numel() * workspace.element_size() < nbytes:
        raise ValueError(f"workspace needs {nbytes} bytes")
    return _ptr(workspace, "workspace"), workspace.numel() * workspace.element_size()


def batched_decode_cu(query, key_cache, value_cache, out, context_lens, max_context_len,
                      kv_head_num, cache_batch_stride=None, cache_tok_stride=None, scale=0.0,
                      split_tokens=0, workspace=None, config=None):
    """Decode one query row per sequence over per-sequence contiguous caches.

    query/out [B, head_num, head_size]; caches [B, max_seq, kv_head_num, head_size]
    unless explicit element strides are given; context_lens int32 [B] on the GPU."""
    B, head_num, head_size = query.shape
    if cache_tok_stride is None:
        cache_tok_stride = kv_head_num * head_size
    if cache_batch_stride is None:
        cache_batch_stride = key_cache.stride(0)
    dt = _dtype(query, key_cache, value_cache, out)
    nbytes = decode_workspace_size(B, head_num, kv_head_num, head_size, max_context_len,
                                   split_tokens)
    wp, wn = _workspace(nbytes, workspace, query.device)
    _lib.check("orin_attn_decode", _lib.load().orin_attn_decode(
        _ptr(query, "query"), _ptr(key_cache, "key_cache"), _ptr(value_cache, "value_cache"),
        _ptr(out, "out"), B, head_num, kv_head_num, head_size, cache_batch_stride,
        cache_tok_stride, _i32(context_lens, "context_lens"), max_context_len, dt, scale,
        split_tokens, wp, wn, _stream(config)))


KV_LAYOUT_TOKEN_MAJOR = 0
KV_LAYOUT_HEAD_MAJOR = 1


def paged_decode_cu(query, k_pool, v_pool, out, block_tables, context_lens, max_context_len,
                    scale=0.0, split_tokens=0, workspace=None, config=None,
                    layout=KV_LAYOUT_TOKEN_MAJOR):
    """Paged decode.  query/out [B, head_num, head_size]; pools
    [num_blocks, block_size, kv_head_num, head_size] (token-major) or
    [num_blocks, kv_head_num, block_size, head_size] (head-major); block_tables int32
    [B, max_blocks]; context_lens int32 [B]."""
    B, head_num, head_size = query.shape
    if layout == KV_LAYOUT_TOKEN_MAJOR:
        _, block_size, kv_head_num, hs2 = k_pool.shape
    else:
        _, kv_head_num, block_size, hs2 = k_pool.shape
    if hs2 != head_size:
        raise ValueError("pool head_size differs from query head_size")
    dt = _dtype(query, k_pool, v_pool, out)
    nbytes = decode_workspace_size(B, head_num, kv_head_num, head_size, max_context_len,
                                   split_tokens)
    wp, wn = _workspace(nbytes, workspace, query.device)
    _lib.check("orin_attn_decode_paged", _lib.load().orin_attn_decode_paged(
        _ptr(query, "query"), _ptr(k_pool, "k_pool"), _ptr(v_pool, "v_pool"), _ptr(out, "out"),
        B, head_num, kv_head_num, head_size, _i32(block_tables, "block_tables"),
        block_tables.shape[1], block_size, layout, _i32(context_lens, "context_lens"),
        max_context_len,
        dt, scale, split_tokens, wp, wn, _stream(config)))


# ---------------------------------------------------------------- vision

def vision_attention_pretransposed_cu(q_trans, k_trans, v_trans, output, out_transposed, scores,
                                      num_tokens, num_heads, head_dim, softmax_scale,
                                      config=None):
    """kernel::vision_attention_pretransposed_cu
    (kuiper/source/op/kernels/cuda/vision_encoder_kernel.cuh:159-170)."""
    dt = _dtype(q_trans, k_trans, v_trans, output)
    _lib.check("orin_vision_attention_pretransposed",
               _lib.load().orin_vision_attention_pretransposed(
                   _ptr(q_trans, "q"), _ptr(k_trans, "k"), _ptr(v_trans, "v"),
                   _ptr(output, "output"), _ptr(out_transposed, "out_transposed"),
                   _ptr(scores, "scores"), num_tokens, num_heads, head_dim,
                   float(softmax_scale), dt, _stream(config)))


def vision_attention_varlen_cu(q_trans, k_trans, v_trans, output, cu_seqlens, max_seqlen,
                               num_heads, head_dim, softmax_scale=0.0, config=None):
    """Varlen vision attention: q/k/v [num_heads, N, head_dim], output [N, num_heads*head_dim],
    cu_seqlens int32 [n_seqs+1] on the GPU."""
    dt = _dtype(q_trans, k_trans, v_trans, output)
    n_seqs = cu_seqlens.numel() - 1
    num_tokens = q_trans.shape[1]
    _lib.check("orin_vision_attention_varlen", _lib.load().orin_vision_attention_varlen(
        _ptr(q_trans, "q"), _ptr(k_trans, "k"), _ptr(v_trans, "v"), _ptr(output, "output"),
        _i32(cu_seqlens, "cu_seqlens"), n_seqs, max_seqlen, num_tokens, num_heads, head_dim,
        float(softmax_scale), dt, _stream(config)))


# ---------------------------------------------------------------- KV-cache writes

KV_TO_PAGED = 0
KV_TO_CONTIGUOUS = 1


def batched_matmul_kernel_cu(input, weight, output, batch_size, scale=1.0, config=None):
    """kernel::batched_matmul_kernel_cu (matmul_kernel.cuh:15-41): output [batch, out_dim] =
    scale * input [batch, in_dim] @ weight[out_dim, in_dim]^T (the wo projection)."""
    out_dim, in_dim = weight.shape
    if input.numel() != batch_size * in_dim or output.numel() != batch_size * out_dim:
        raise ValueError("input / output sizes do not match the weight")
    dt = _dtype(input, weight, output)
    _lib.check("orin_batched_matmul", _lib.load().orin_batched_matmul(
        _ptr(input, "input"), _ptr(weight, "weight"), _ptr(output, "output"), batch_size, in_dim,
        out_dim, float(scale), dt, _stream(config)))


def copy_to_kv_cache_kernel(kv_cache, src, pos, kv_dim, layer_idx, seq_len, config=None):
    """kernel::copy_to_kv_cache_kernel / copy_to_kv_cache_kernel_fp16
    (kuiper/source/op/kernels/cuda/kv_cache_kernel.cuh:24-33): src [kv_dim] goes to row
    *pos of layer layer_idx of kv_cache [layers, seq_len, kv_dim]; pos is an int32 GPU
    tensor read when the kernel runs."""
    dt = _dtype(kv_cache, src)
    _lib.check("orin_copy_to_kv_cache", _lib.load().orin_copy_to_kv_cache(
        _ptr(kv_cache, "kv_cache"), _ptr(src, "src"), _i32(pos, "pos"), kv_dim, layer_idx,
        seq_len, dt, _stream(config)))


def kv_cache_write_paged(k_src, v_src, k_pool, v_pool, slot_mapping,
                         layout=KV_LAYOUT_TOKEN_MAJOR, config=None):
    """Store rows of k_src / v_src [n, kv_heads, head_size] at pool slots slot_mapping
    (int32 [n], block * block_size + offset; negative = skip)."""
    n, kv_heads, head_size = k_src.shape
    if layout == KV_LAYOUT_TOKEN_MAJOR:
        _, block_size, hkv, hs = k_pool.shape
    else:
        _, hkv, block_size, hs = k_pool.shape
    if (hkv, hs) != (kv_heads, head_size) or v_src.shape != k_src.shape:
        raise ValueError("pool and source shapes disagree")
    dt = _dtype(k_src, v_src, k_pool, v_pool)
    _lib.check("orin_kv_cache_write_paged", _lib.load().orin_kv_cache_write_paged(
        _ptr(k_src, "k_src"), _ptr(v_src, "v_src"), kv_heads * head_size, _ptr(k_pool, "k_pool"),
        _ptr(v_pool, "v_pool"), _i32(slot_mapping, "slot_mapping"), n, kv_heads, head_size,
        block_size, layout, dt, _stream(config)))


def kv_cache_convert(contig, pool, block_table, n_tokens, direction,
                     layout=KV_LAYOUT_TOKEN_MAJOR, config=None):
    """Copy tokens [0, n_tokens) of one sequence between contig [>= n_tokens, kv_heads,
    head_size] and a paged pool through block_table (int32 [max_blocks])."""
    _, kv_heads, head_size = contig.shape
    block_size = pool.shape[1] if layout == KV_LAYOUT_TOKEN_MAJOR else pool.shape[2]
    dt = _dtype(contig, pool)
    _lib.check("orin_kv_cache_convert", _lib.load().orin_kv_cache_convert(
        _ptr(contig, "contig"), kv_heads * head_size, _ptr(pool, "pool"),
        _i32(block_table, "block_table"), n_tokens, kv_heads, head_size, block_size, layout,
        direction, dt, _stream(config)))


# ---------------------------------------------------------------- Q/K producers

def sin_cos_cache_calc_cu(head_size, max_seq_len, sin_cache, cos_cache, theta=1e6, config=None):
    """kernel::sin_cos_cache_calc_cu (kuiper/source/op/kernels/cuda/rope_kernel.cu:153-166):
    fp32 [max_seq_len, head_size] tables, entry [p][i] = sin/cos(p * theta^(-i/head_size))."""
    if sin_cache.dtype != torch.float32 or cos_cache.dtype != torch.float32:
        raise ValueError("sin/cos caches are fp32")
    _lib.check("orin_rope_sin_cos_cache", _lib.load().orin_rope_sin_cos_cache(
        _ptr(sin_cache, "sin_cache"), _ptr(cos_cache, "cos_cache"), head_size, max_seq_len,
        float(theta), _stream(config)))


def qk_norm_rope_cu(query, key, value, q_norm_weight, k_norm_weight, sin_cache, cos_cache,
                    key_cache, value_cache, layer_index, max_seq_len, start_pos, seq_len,
                    head_num, kv_head_num, head_size, eps=1e-6, pos_ptr=None, config=None):
    """The Qwen3 producer in one pass: per-head RMSNorm + RoPE of query (in place) and key,
    key and value rows stored at positions start_pos.. of layer layer_index of the kuiper
    caches.  q/k_norm_weight may be None (no normalisation).  pos_ptr (int32 GPU tensor)
    replaces start_pos when given."""
    dt = _dtype(*[x for x in (query,) if x is not None], key, value, key_cache, value_cache,
                *[w for w in (q_norm_weight, k_norm_weight) if w is not None])
    _lib.check("orin_qk_norm_rope", _lib.load().orin_qk_norm_rope(
        _ptr(query, "query"), _ptr(key, "key"), _ptr(value, "value"),
        _ptr(q_norm_weight, "q_norm_weight"), _ptr(k_norm_weight, "k_norm_weight"),
        _ptr(sin_cache, "sin_cache"), _ptr(cos_cache, "cos_cache"), _ptr(key_cache, "key_cache"),
        _ptr(value_cache, "value_cache"), layer_index, max_seq_len, start_pos,
        None if pos_ptr is None else _i32(pos_ptr, "pos_ptr"), seq_len, head_num, kv_head_num,
        head_size, float(eps), dt, _stream(config)))


def fused_split_rope_transpose_cu(qkv, cos_cache, sin_cache, q_trans, k_trans, v_trans,
                                  num_tokens, num_heads, head_dim, config=None):
    """kernel::fused_split_rope_transpose_cu
    (kuiper/source/op/kernels/cuda/vision_encoder_kernel.cu:752-773)."""
    dt = _dtype(qkv, cos_cache, sin_cache, q_trans, k_trans, v_trans)
    _lib.check("orin_vision_split_rope_transpose",
               _lib.load().orin_vision_split_rope_transpose(
                   _ptr(qkv, "qkv"), _ptr(cos_cache, "cos_cache"), _ptr(sin_cache, "sin_cache"),
                   _ptr(q_trans, "q_trans"), _ptr(k_trans, "k_trans"), _ptr(v_trans, "v_trans"),
                   num_tokens, num_heads, head_dim, dt, _stream(config)))
