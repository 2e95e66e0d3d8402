"""Torch-tensor front end of the C-ABI (the host-side mirror of the reference launches).

Names follow the reference kernels each call replaces.  Tensors must live on the GPU
(except RopeTable, which builds a host table as the reference does); BF16 activations
are torch.bfloat16 (or int16 views of BF16 bits), fp32 activations torch.float32.
Every call is asynchronous on the current torch stream and raises PadraError on a
nonzero status.  Device-detected problems set the caller's `bad` flag (int32 tensor).
"""
from __future__ import annotations

import ctypes

import torch

from . import abi

_BF16_DTYPES = (torch.bfloat16, torch.int16, torch.uint16)


def _act(t: torch.Tensor) -> int:
    if t.dtype in _BF16_DTYPES:
        return abi.ACT_BF16
    if t.dtype == torch.float32:
        return abi.ACT_F32
    raise TypeError(f"activation dtype {t.dtype} (want bfloat16 or float32)")


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _need_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("padra_amd ops take GPU tensors")


def ResidualPostNorm(x, residual, normalized, gamma, bad, eps=1e-6, tree=abi.TREE_128,
                     statistics=None):
    """x <- B(x + residual); normalized <- B(B(x*inv)*gamma).  residual=None: RMSNorm only.

    Replaces ResidualPostNormWideExact (tree=256), Add+Norm (tree=128)
    (residual_norm_wide_exact.cuh:6-80, inference.cu:188-214, 475-481).
    """
    _need_cuda(x, residual, normalized, gamma, bad, statistics)
    rows, hidden = x.shape[0], x.shape[-1]
    abi.call("padra_ResidualPostNorm", _stream(x), _p(x), _p(residual), _p(normalized),
             _p(gamma), rows, hidden, float(eps), int(tree), _p(statistics), _p(bad), _act(x))


def NormFP8(x, normalized, gamma, packed, scales, bad, eps=1e-6, statistics=None):
    """normalized <- 128-thread RMSNorm of x; packed <- E4M3 codes of normalized/scale,
    scales[row] = max|normalized|/448 (NormFP8Exact, norm_fp8_exact.cuh:6-62)."""
    _need_cuda(x, normalized, gamma, packed, scales, bad, statistics)
    rows, hidden = x.shape[0], x.shape[-1]
    abi.call("padra_NormFP8", _stream(x), _p(x), _p(normalized), _p(gamma), _p(packed),
             _p(scales), rows, hidden, float(eps), _p(statistics), _p(bad), _act(x))


def QuantizeFP8(x, packed, scales, bad):
    """packed <- E4M3 codes of x/scale, scales[row] = max|x|/448 (QuantizeFP8,
    prefill.cuh:46-66)."""
    _need_cuda(x, packed, scales, bad)
    abi.call("padra_QuantizeFP8", _stream(x), _p(x), _p(packed), _p(scales), x.shape[0],
             x.shape[-1], _p(bad), _act(x))


def Combine(x, down, weights, bad, residual=True):
    """x <- [B(x + c) | c], c the ordered BF16 combine of the 8 expert rows
    (Combine, inference.cu:580-590).  down [rows][8][hidden], weights [rows][8] fp32."""
    _need_cuda(x, down, weights, bad)
    rows, hidden = x.shape[0], x.shape[-1]
    abi.call("padra_Combine", _stream(x), _p(x), _p(down), _p(weights), rows, hidden,
             down.shape[1], int(bool(residual)), _p(bad), _act(x))


def CombineNorm(x, down, weights, normalized, gamma, bad, packed=None, scales=None, eps=1e-6,
                statistics=None):
    """Residual combine, then RMSNorm (+ FP8 when packed is given)
    (combine_norm_exact::CombineNorm, combine_norm_exact.cuh:7-72)."""
    _need_cuda(x, down, weights, normalized, gamma, bad, packed, scales, statistics)
    rows, hidden = x.shape[0], x.shape[-1]
    abi.call("padra_CombineNorm", _stream(x), _p(x), _p(down), _p(weights), _p(normalized),
             _p(gamma), _p(packed), _p(scales), rows, hidden, down.shape[1], float(eps),
             _p(statistics), _p(bad), _act(x))


def RopeTable(positions, head_dim=128, theta=1e6, yarn=False, factor=16.0,
              original_context=8192) -> torch.Tensor:
    """Host BF16 cos|sin table [positions][head_dim] (RopeTable, inference.cu:764-785)."""
    out = torch.empty((positions, head_dim), dtype=torch.int16)
    abi.call("padra_RopeTable", _p(out), int(positions), int(head_dim), float(theta),
             int(bool(yarn)), float(factor), int(original_context))
    return out.view(torch.bfloat16)


def positions_base(base: int = 0) -> abi.Positions:
    return abi.Positions(mode=abi.POS_BASE, base=int(base), prefill=None, decode=None,
                         maximum=131072, vocab=98304, binding_epoch=1)


def positions_prefill(state: torch.Tensor, maximum=131072, binding_epoch=1) -> abi.Positions:
    """state: device int32[8] holding a PrefillState (kept alive by the returned object)."""
    p = abi.Positions(mode=abi.POS_PREFILL, base=0, prefill=state.data_ptr(), decode=None,
                      maximum=int(maximum), vocab=98304, binding_epoch=int(binding_epoch))
    p._keep = state
    return p


def positions_decode(states: torch.Tensor, maximum=131072, vocab=98304) -> abi.Positions:
    """states: device int32[n][8], one DecodeState per sequence (kept alive by the result)."""
    p = abi.Positions(mode=abi.POS_DECODE, base=0, prefill=None, decode=states.data_ptr(),
                      maximum=int(maximum), vocab=int(vocab), binding_epoch=1)
    p._keep = states
    return p


def kv_cache(fmt, k, v, cap, scales=None, first=0, seq_stride=0) -> abi.KVCache:
    """A cache binding; the returned object keeps k, v and scales alive."""
    c = abi.KVCache(format=int(fmt), k=k.data_ptr(), v=v.data_ptr(),
                    scales=None if scales is None else scales.data_ptr(), cap=int(cap),
                    first=int(first), seq_stride=int(seq_stride))
    c._keep = (k, v, scales)
    return c


def q8_0_row_bytes(features: int) -> int:
    """CacheRow size: fp16 d[F/32] + int8 qs[F], 16-byte aligned (kv_q8_layout.cuh:6-12)."""
    return (2 * (features // 32) + features + 15) // 16 * 16


def kv_cache_layout(fmt: int, rows: int, features: int = 512) -> dict:
    """Byte offsets of one layer's cache, KVCacheLayout::Make (kv_cache_layout.h:12-33)."""
    if not 1 <= rows <= 131072:
        raise ValueError("unsupported KV row capacity")
    if fmt == abi.KV_BF16:
        return {"v_offset": rows * 2 * features, "scales_offset": 0, "bytes": rows * 4 * features}
    if fmt == abi.KV_Q8:
        heads = features // 128
        return {"v_offset": rows * features, "scales_offset": rows * 2 * features,
                "bytes": rows * (2 * features + 8 * heads)}
    if fmt in (abi.KV_Q8_0, abi.KV_Q8_0_NOROT):
        rb = q8_0_row_bytes(features)
        return {"v_offset": rows * rb, "scales_offset": 0, "bytes": rows * 2 * rb}
    raise ValueError("unknown KV format")


def _shape_qk(q, k):
    tokens, q_heads, head_dim = q.shape
    if k.shape[0] != tokens or k.shape[2] != head_dim:
        raise ValueError("q [T][Hq][D] and k [T][Hkv][D] disagree")
    return tokens, q_heads, k.shape[1], head_dim


def QKNormRopeStore(q, k, qn, kn, table, positions: abi.Positions, bad, eps=1e-6, v=None,
                    kv: abi.KVCache | None = None):
    """Per-head RMSNorm + NeoX RoPE of q [T][Hq][D], k [T][Hkv][D] in place; with kv, the
    rotated K rows and V rows are stored at slot position % cap.

    Replaces QKNormRope / QKNormRopePair64 / QKNormRopeControlled /
    QKNormRopeStoreControlled and the cache writers after them (see padra_hip.h).
    """
    _need_cuda(q, k, v, qn, kn, table, bad)
    tokens, q_heads, kv_heads, head_dim = _shape_qk(q, k)
    abi.call("padra_QKNormRopeStore", _stream(q), _p(q), _p(k), _p(v), _p(qn), _p(kn),
             _p(table), table.shape[0], ctypes.byref(positions), tokens, q_heads, kv_heads,
             head_dim, float(eps), None if kv is None else ctypes.byref(kv), _p(bad), _act(q))


def ResidualNormQKRopeStore(x, residual, normalized, gamma, q, k, v, qn, kn, table,
                            positions: abi.Positions, kv: abi.KVCache | None, bad, eps=1e-6,
                            tree=abi.TREE_128, statistics=None):
    """ResidualPostNorm and QKNormRopeStore over the same tokens in one launch (BF16 or
    fp32 activations, by x's dtype)."""
    _need_cuda(x, residual, normalized, gamma, q, k, v, qn, kn, table, bad, statistics)
    tokens, q_heads, kv_heads, head_dim = _shape_qk(q, k)
    if x.shape[0] != tokens:
        raise ValueError("x rows must equal the token count")
    abi.call("padra_ResidualNormQKRopeStore", _stream(x), _p(x), _p(residual), _p(normalized),
             _p(gamma), x.shape[-1], int(tree), _p(statistics), _p(q), _p(k), _p(v), _p(qn),
             _p(kn), _p(table), table.shape[0], ctypes.byref(positions), tokens, q_heads,
             kv_heads, head_dim, float(eps), None if kv is None else ctypes.byref(kv), _p(bad),
             _act(x))


def EmbedResidualNormQKRopeStore(embed, ids, x, residual, normalized, gamma, q, k, v, qn, kn,
                                 table, positions: abi.Positions, kv: abi.KVCache | None, bad,
                                 eps=1e-6, tree=abi.TREE_256, statistics=None):
    """Embed (x <- embed[token]) then ResidualNormQKRopeStore, in one launch."""
    _need_cuda(embed, ids, x, residual, normalized, gamma, q, k, v, qn, kn, table, bad, statistics)
    tokens, q_heads, kv_heads, head_dim = _shape_qk(q, k)
    if x.shape[0] != tokens or embed.shape[-1] != x.shape[-1]:
        raise ValueError("x rows must equal the token count and embed rows x's width")
    abi.call("padra_EmbedResidualNormQKRopeStore", _stream(x), _p(embed), embed.shape[0],
             _p(ids), _p(x), _p(residual), _p(normalized), _p(gamma), x.shape[-1], int(tree),
             _p(statistics), _p(q), _p(k), _p(v), _p(qn), _p(kn), _p(table), table.shape[0],
             ctypes.byref(positions), tokens, q_heads, kv_heads, head_dim, float(eps),
             None if kv is None else ctypes.byref(kv), _p(bad))


def KVStore(k, v, positions: abi.Positions, kv: abi.KVCache, bad):
    """Store / encode K [T][Hkv][D] (already rotated) and V rows into the cache."""
    _need_cuda(k, v, bad)
    tokens, kv_heads, head_dim = k.shape
    abi.call("padra_KVStore", _stream(k), _p(k), _p(v), ctypes.byref(positions), tokens,
             kv_heads, head_dim, ctypes.byref(kv), _p(bad), _act(k))


def KVCommit(chunk: abi.KVCache, ring: abi.KVCache, positions: abi.Positions, tokens, kv_heads,
             bad):
    """Copy encoded chunk rows r >= ring.first to ring slots position(r) % ring.cap."""
    _need_cuda(bad)
    abi.call("padra_KVCommit", _stream(bad), ctypes.byref(chunk), ctypes.byref(ring),
             ctypes.byref(positions), int(tokens), int(kv_heads), _p(bad))


def KvQ8_0Dequantize(rows_k, rows_v, out_k, out_v, bad, kv_heads=4):
    _need_cuda(rows_k, rows_v, out_k, out_v, bad)
    abi.call("padra_KvQ8_0Dequantize", _stream(out_k), _p(rows_k), _p(rows_v), _p(out_k),
             _p(out_v), rows_k.shape[0], int(kv_heads), _p(bad), _act(out_k))


def KvQ8_0DequantizePrefix(rows_k, rows_v, out_k, out_v, positions: abi.Positions, tokens, bad,
                           kv_heads=4):
    """Decode the ring's first min(base, cap) rows (cap = rows_k.shape[0]) to BF16."""
    _need_cuda(rows_k, rows_v, out_k, out_v, bad)
    abi.call("padra_KvQ8_0DequantizePrefix", _stream(out_k), _p(rows_k), _p(rows_v), _p(out_k),
             _p(out_v), ctypes.byref(positions), int(tokens), rows_k.shape[0], int(kv_heads),
             _p(bad))


def KVCheckpointCapture(ring: abi.KVCache, chunk: abi.KVCache, saved: abi.KVCache,
                        positions: abi.Positions, tokens, anchor, bad, kv_heads=4):
    """Snapshot of a 1024-row local ring at `anchor` (kv_checkpoint.cuh:27-89)."""
    _need_cuda(bad)
    abi.call("padra_KVCheckpointCapture", _stream(bad), ctypes.byref(ring), ctypes.byref(chunk),
             ctypes.byref(saved), ctypes.byref(positions), int(tokens), int(anchor),
             int(kv_heads), _p(bad))


def DecodeAttention(q, kv: abi.KVCache, out, positions: abi.Positions, bad, kv_heads=4,
                    local=False, splits=0, scratch=None, packed=None, scales=None):
    """Decode attention over a BF16 or q8_0 cache for q [seqs][q_heads][128]
    (SplitBF16 + per-head Merge, attention_gqa8_fragment_validation.cuh:79-214,
    attention_perhead_exact.cuh:7-38; q8_native EncodeQuery/Split/Merge,
    kv_q8_native.cuh:103-363).  splits: 0 runs the reference's split count, -1 the MI355X-tuned
    count (fewer splits for a local ring with many sequences), 1..32 as given; anything else
    raises ValueError.  Allocates the fp32 scratch when none is given.  With packed
    ([seqs][q_heads * 128] uint8) and scales ([seqs] fp32), the merge also writes each
    output row's E4M3 encoding (MergeQuantize, attention_merge_quantize_wide_exact.cuh:9-66)."""
    _need_cuda(q, out, bad, scratch)
    seqs, q_heads = q.shape[0], q.shape[1]
    used = abi.lib().padra_DecodeAttentionSplits(ctypes.byref(kv), seqs, int(kv_heads),
                                                 int(bool(local)), int(splits))
    if used < 1:
        raise ValueError("invalid decode attention arguments")
    need = abi.lib().padra_DecodeAttentionScratch(kv.format, seqs, q_heads, used)
    if scratch is None:
        scratch = torch.empty(need, dtype=torch.float32, device=q.device)
    if packed is None:
        abi.call("padra_DecodeAttention", _stream(q), _p(q), ctypes.byref(kv), _p(out),
                 ctypes.byref(positions), seqs, q_heads, int(kv_heads), int(bool(local)),
                 int(splits), _p(scratch), scratch.numel(), _p(bad), _act(q))
    else:
        _need_cuda(packed, scales)
        abi.call("padra_DecodeAttentionFP8", _stream(q), _p(q), ctypes.byref(kv), _p(out),
                 _p(packed), _p(scales), ctypes.byref(positions), seqs, q_heads, int(kv_heads),
                 int(bool(local)), int(splits), _p(scratch), scratch.numel(), _p(bad), _act(q))
    return scratch


def RotateRows(data, bad, value=False):
    """In-place Hadamard rotation of 128-wide rows (K transform, or V with value=True)."""
    _need_cuda(data, bad)
    abi.call("padra_RotateRows", _stream(data), _p(data), data.numel() // 128, int(bool(value)),
             _p(bad), _act(data))


def SiluTableBuild(table):
    """table: device int16/uint16 [65536]."""
    _need_cuda(table)
    abi.call("padra_SiluTableBuild", _stream(table), _p(table))


def SwiGLU(gate, up, out, table, bad):
    _need_cuda(gate, up, out, table, bad)
    abi.call("padra_SwiGLU", _stream(gate), _p(gate), _p(up), _p(out), gate.numel(), _p(table),
             _p(bad), _act(gate))


def Embed(table, out, bad, ids=None, positions: abi.Positions | None = None, tokens=None):
    """out[t] = table[token_t]; token from ids, a PrefillState prompt or DecodeStates."""
    _need_cuda(table, out, bad, ids)
    vocab, hidden = table.shape
    tokens = out.shape[0] if tokens is None else tokens
    abi.call("padra_Embed", _stream(out), _p(table), vocab, hidden, _p(ids),
             None if positions is None else ctypes.byref(positions), int(tokens), _p(out),
             _p(bad), _act(out))
