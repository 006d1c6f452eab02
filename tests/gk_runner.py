"""Call the C ABI (libgaudirt_amd.so) on torch device buffers, for the GPU tests."""

import ctypes

import numpy as np
import torch

from gaudirt_amd import capi


def to_device(array, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(array))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def bf16_device(bits):
    return to_device(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16), torch.bfloat16)


def bits_of(tensor):
    return tensor.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def decode_params(query, pool, tables, lens, heads, kv_heads, head_dim, block_size, scale, out, *,
                  row_request=None, max_context=None, partition=0, softcap=0.0, window=-1,
                  new_key=None, new_value=None, slot_mapping=None):
    p = capi.DecodeParams()
    p.query = query.data_ptr()
    p.q_row_stride = query.stride(0)
    p.pool = pool.data_ptr()
    p.slots = pool.shape[2]
    p.block_tables = tables.data_ptr()
    p.bt_stride = tables.stride(0)
    p.block_size = block_size
    p.row_request = row_request.data_ptr() if row_request is not None else None
    p.row_context = lens.data_ptr()
    p.rows = query.shape[0]
    p.q_heads, p.kv_heads, p.head_dim = heads, kv_heads, head_dim
    p.scale, p.softcap, p.sliding_window = scale, softcap, window
    p.max_context = int(max_context if max_context is not None else lens.max().item())
    p.partition_tokens = partition
    p.out = out.data_ptr()
    p.out_row_stride = out.stride(0)
    if new_key is not None:
        p.new_key = new_key.data_ptr()
        p.new_value = new_value.data_ptr()
        p.new_kv_row_stride = new_key.stride(0)
        p.slot_mapping = slot_mapping.data_ptr()
    return p


def paged_decode(params):
    lib = capi.load()
    need = lib.gk_paged_decode_workspace_bytes(ctypes.byref(params))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    capi.check(lib.gk_paged_decode(ctypes.byref(params), ctypes.c_void_p(ws.data_ptr()), need,
                                   capi.current_stream()))
    return ws


def run_case(case, partition=0, out=None):
    """Run gk_paged_decode on a host DecodeCase; returns output bf16 bits [B, Hq*d]."""
    q = bf16_device(case.query)
    pool = bf16_device(case.pool)
    tables = to_device(case.block_tables)
    lens = to_device(case.lens.astype(np.int32))
    out = torch.full((case.batch, case.heads * case.head_dim), float("nan"), dtype=torch.bfloat16, device="cuda")
    params = decode_params(q, pool, tables, lens, case.heads, case.kv_heads, case.head_dim, case.block_size,
                           case.scale, out, partition=partition, softcap=case.softcap, window=case.window)
    ws = paged_decode(params)
    torch.cuda.synchronize()
    del ws
    return bits_of(out)


def kv_store(key, value, slot_mapping, pool, kv_heads, head_dim):
    lib = capi.load()
    capi.check(lib.gk_kv_store(ctypes.c_void_p(key.data_ptr()), ctypes.c_void_p(value.data_ptr()), key.stride(0),
                               value.stride(0), ctypes.c_void_p(slot_mapping.data_ptr()), key.shape[0],
                               ctypes.c_void_p(pool.data_ptr()), pool.shape[2], kv_heads, head_dim,
                               capi.current_stream()))


def prefill_params(query, pool, tables, seq_request, seq_first_row, seq_rows, seq_prefix, heads, kv_heads,
                   head_dim, block_size, scale, out, max_rows, softcap=0.0, window=-1):
    p = capi.PrefillParams()
    p.query, p.q_row_stride = query.data_ptr(), query.stride(0)
    p.pool, p.slots = pool.data_ptr(), pool.shape[2]
    p.block_tables, p.bt_stride, p.block_size = tables.data_ptr(), tables.stride(0), block_size
    p.seq_request, p.seq_first_row = seq_request.data_ptr(), seq_first_row.data_ptr()
    p.seq_rows, p.seq_prefix = seq_rows.data_ptr(), seq_prefix.data_ptr()
    p.seqs, p.max_rows = seq_rows.shape[0], max_rows
    p.q_heads, p.kv_heads, p.head_dim = heads, kv_heads, head_dim
    p.scale, p.softcap, p.sliding_window = scale, softcap, window
    p.out, p.out_row_stride = out.data_ptr(), out.stride(0)
    return p


def run_prefill_case(case):
    """Run gk_paged_prefill on a paged_cases.PrefillCase; returns output bf16 bits [rows, Hq*d]."""
    q = bf16_device(case.query)
    pool = bf16_device(case.pool)
    tables = to_device(case.block_tables)
    seqs = len(case.chunks)
    out = torch.full((case.rows, case.heads * case.head_dim), float("nan"), dtype=torch.bfloat16, device="cuda")
    params = prefill_params(q, pool, tables, to_device(np.arange(seqs, dtype=np.int32)), to_device(case.first_rows),
                            to_device(case.chunks), to_device(case.prefixes), case.heads, case.kv_heads,
                            case.head_dim, case.block_size, case.scale, out, int(case.chunks.max()),
                            case.softcap, case.window)
    capi.check(capi.load().gk_paged_prefill(ctypes.byref(params), capi.current_stream()))
    torch.cuda.synchronize()
    return bits_of(out)
