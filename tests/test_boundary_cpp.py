"""The C-ABI header compiled as C++20 next to the reference's own host headers (CPU only).

- static_asserts that padra_PrefillState, padra_DecodeState and padra_Q8KVScalePair have
  the size, field offsets and field types of mellum16::PrefillState
  (src/runtime/prefill_state.h:6-10), DecodeState (src/cuda/decode_control.cuh:3-6) and
  mellum16::Q8KVScalePair (src/runtime/kv_cache_layout.h:48-51), and that the PADRA_KV_*
  codes follow mellum16::KVCacheFormat's order (kv_cache_layout.h:6);
- runs mellum16::KVCacheLayout::Make for every format at 1, 1024, 8192 and 131072 rows and
  compares it with padra_amd.ops.kv_cache_layout, which the tests and the bench use;
- compiles the C++ calls of the repository's integration guide (its section 1) with
  -fsyntax-only against include/padra_hip.h.

The reference headers are read where they lie under /root/reference (nothing is copied
into the repository); DecodeState lives in a CUDA header, so its struct definition is
extracted from that file at test time.  Skipped when the reference or g++ is absent (the
GPU box has neither the reference nor needs it).
"""
import os
import re
import shutil
import subprocess

import pytest

from padra_amd import abi, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference/src"

pytestmark = pytest.mark.skipif(
    not os.path.isdir(os.path.join(REF, "runtime")) or shutil.which("g++") is None,
    reason="needs the reference's host headers and g++")


def _decode_state_definition() -> str:
    text = open(os.path.join(REF, "cuda", "decode_control.cuh")).read()
    m = re.search(r"struct DecodeState \{[^}]*\};", text)
    assert m, "DecodeState definition not found in decode_control.cuh"
    return m.group(0)


LAYOUT_TU = r'''
#include <cstddef>
#include <cstdio>
#include <type_traits>
#include "padra_hip.h"
#include "runtime/kv_cache_layout.h"
#include "runtime/prefill_state.h"
#include "decode_state_ref.h"

#define SAME_FIELD(A, B, F)                                                         \
  static_assert(offsetof(A, F) == offsetof(B, F), #F " offset");                  \
  static_assert(sizeof(A::F) == sizeof(B::F), #F " size");                        \
  static_assert(std::is_signed_v<decltype(A::F)> == std::is_signed_v<decltype(B::F)>, \
                #F " signedness")

using RP = mellum16::PrefillState;
using PP = padra_PrefillState;
static_assert(sizeof(RP) == sizeof(PP) && alignof(RP) == alignof(PP));
SAME_FIELD(RP, PP, base);
SAME_FIELD(RP, PP, prompt_offset);
SAME_FIELD(RP, PP, tokens);
SAME_FIELD(RP, PP, capacity);
SAME_FIELD(RP, PP, committed);
SAME_FIELD(RP, PP, binding_epoch);
SAME_FIELD(RP, PP, request_epoch);
SAME_FIELD(RP, PP, valid);

using RD = DecodeState;
using PD = padra_DecodeState;
static_assert(sizeof(RD) == sizeof(PD) && alignof(RD) == alignof(PD));
SAME_FIELD(RD, PD, token);
SAME_FIELD(RD, PD, position);
SAME_FIELD(RD, PD, capacity);
SAME_FIELD(RD, PD, remaining);
SAME_FIELD(RD, PD, global_valid);
SAME_FIELD(RD, PD, local_valid);
SAME_FIELD(RD, PD, eos);
SAME_FIELD(RD, PD, stopped);

using RS = mellum16::Q8KVScalePair;
using PS = padra_Q8KVScalePair;
static_assert(sizeof(RS) == sizeof(PS));
SAME_FIELD(RS, PS, k);
SAME_FIELD(RS, PS, v);

static_assert(static_cast<int>(mellum16::KVCacheFormat::BF16) == PADRA_KV_BF16);
static_assert(static_cast<int>(mellum16::KVCacheFormat::Q8TokenHead128F32ScaleV1) == PADRA_KV_Q8);
static_assert(static_cast<int>(mellum16::KVCacheFormat::Q8Token512Block32F16ScaleRotatedV2) ==
              PADRA_KV_Q8_0);

int main() {
  const mellum16::KVCacheFormat formats[] = {
      mellum16::KVCacheFormat::BF16, mellum16::KVCacheFormat::Q8TokenHead128F32ScaleV1,
      mellum16::KVCacheFormat::Q8Token512Block32F16ScaleRotatedV2};
  const int rows[] = {1, 1024, 8192, 131072};
  for (auto f : formats)
    for (int r : rows) {
      const auto l = mellum16::KVCacheLayout::Make(f, r);
      std::printf("%d %d %zu %zu %zu %zu %s\n", static_cast<int>(f), r, l.k_offset, l.v_offset,
                  l.scales_offset, l.bytes, l.name());
    }
  return 0;
}
'''


def test_structs_and_layouts_match_reference_headers(tmp_path):
    (tmp_path / "decode_state_ref.h").write_text(
        "#pragma once\n// extracted at test time from decode_control.cuh:3-6\n" +
        _decode_state_definition() + "\n")
    src = tmp_path / "layout.cpp"
    src.write_text(LAYOUT_TU)
    exe = tmp_path / "layout"
    res = subprocess.run(["g++", "-std=c++20", "-Wall", "-Werror", "-I", str(tmp_path), "-I",
                          os.path.join(ROOT, "include"), "-I", REF, "-o", str(exe), str(src)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    lines = out.strip().splitlines()
    assert len(lines) == 12
    names = {abi.KV_BF16: "bf16", abi.KV_Q8: "q8_token_head128_f32scale_v1",
             abi.KV_Q8_0: "q8_0_token512_block32_f16scale_rot_k128_v64_v2"}
    for line in lines:
        fmt, rows, k_off, v_off, s_off, nbytes, name = line.split()
        fmt, rows = int(fmt), int(rows)
        mine = ops.kv_cache_layout(fmt, rows)
        assert int(k_off) == 0
        assert (int(v_off), int(s_off), int(nbytes)) == \
            (mine["v_offset"], mine["scales_offset"], mine["bytes"]), line
        assert name == names[fmt]


def _integration_blocks():
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = text[text.index("## 1."):text.index("## 2.")]
    return re.findall(r"```cpp\n(.*?)```", sec, re.S)


# Declarations of the names the integration guide's snippets use, with the types the
# reference's runtime gives them (fp32 activation buffers, BF16 weights and tables, device states).
SNIPPET_PRELUDE = r'''
#include <algorithm>
#include <cstdint>
#include "padra_hip.h"
struct Stream { void *s; };
struct Q8Planes { void *k, *v; };
struct LayerArgs { void *kc, *vc; int cap; Q8Planes q8; };
static void check(int) {}
void integration_calls(Stream stream, LayerArgs a, float *q, float *k, float *v,
                       const uint16_t *qn_bf16, const uint16_t *kn_bf16,
                       const uint16_t *rope_bf16, int rope_rows, const void *activeState,
                       int contextMaximum, float *x, float *residual, float *normalized,
                       const uint16_t *post_bf16, float *stats, int *bad,
                       const padra_PrefillState *prefill, bool local, int n, float *bq,
                       float *bk, float *bv, const uint16_t *qn, const uint16_t *kn,
                       const uint16_t *rope, float *bx, float *br, float *bn,
                       const uint16_t *norm_bf16, uint8_t *fp8Input, float *fp8Scales,
                       float *attn, uint8_t *attnFp8, float *attnScales, float *down,
                       const float *routing, int rows, float *gate, float *up,
                       const uint16_t *silu_table, bool q8Native, void *kc, void *vc,
                       float *fastAttentionScratch, long long scratch_floats, void *kc8,
                       void *vc8, void *q8Scales, float *attnScale, const uint16_t *embed_bf16,
                       float *r, void *ring_k, void *ring_v, void *out_k, void *out_v) {
'''


def test_integration_snippets_compile(tmp_path):
    blocks = _integration_blocks()
    assert len(blocks) >= 2
    body = "\n".join(b.replace('#include "padra_hip.h"', "") for b in blocks)
    src = tmp_path / "calls.cpp"
    src.write_text(SNIPPET_PRELUDE + body + "\n}\n")
    res = subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-Wno-unused-variable",
                          "-I", os.path.join(ROOT, "include"), str(src)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
