"""The drop-in boundary without a GPU: C-ABI exports and argument checks,
the Python mirror's validation (order, exception types, messages), the
workspace capacity contract and the byte models used by the benchmark.

Nothing here launches a kernel: C-ABI calls are made only with arguments the
library rejects before touching the device.
"""

from __future__ import annotations

import ctypes
import json
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from tensorforge_amd import _native
from tensorforge_amd.kernels import (
    PagedAttentionWorkspace,
    argmax_rows,
    autotune_cache_size,
    paged_gqa_decode_attention,
    paged_kv_write_slots,
    paged_kv_write_token,
    residual_rms_norm,
    rms_norm,
    selected_autotune_config,
    set_attention_split_size,
    swiglu,
)
from tensorforge_amd.kernels.attention import (
    attention_plan,
    attention_split_size,
    attention_split_size_for,
)
from tensorforge_amd.workloads import (
    decode_attention_bytes,
    kv_append_bytes,
    make_decode_attention_case,
    rms_norm_bytes,
    swiglu_bytes,
    tinyllama_decode_case,
    tinyllama_decode_lengths,
)

REPO_ROOT = Path(__file__).resolve().parents[1]
HEADER = REPO_ROOT / "include" / "tensorforge_amd.h"


@pytest.fixture(scope="module")
def lib() -> ctypes.CDLL:
    if not _native.LIBRARY_PATH.exists():
        from tensorforge_amd import build

        build.build()
    return _native.library()


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"\b(tf_[a-z0-9_]+)\s*\(", text)


def test_library_exports_every_declared_symbol(lib) -> None:
    declared = _declared_functions()
    assert len(declared) == len(set(declared)) >= 10
    for name in declared:
        assert hasattr(lib, name), f"{name} is declared in the header but not exported"
    assert set(declared) == set(_native.SIGNATURES), "ctypes signatures and header disagree"


def test_header_constants_match_the_python_binding() -> None:
    text = HEADER.read_text()
    for name in ("TF_ATTENTION_FLAG_FORCE_GENERIC",
                 "TF_ATTENTION_FLAG_VALU", "TF_ATTENTION_FLAG_BALANCED",
                 "TF_ATTENTION_WAVES_PER_CU_SHIFT",
                 "TF_ATTENTION_HEADS_PER_WG_SHIFT", "TF_ATTENTION_TOKENS_PER_WAVE_SHIFT"):
        match = re.search(rf"#define {name} (\d+)", text)
        assert match and int(match.group(1)) == getattr(_native, name), name
    for name in ("TF_DTYPE_FLOAT32", "TF_DTYPE_FLOAT16", "TF_DTYPE_BFLOAT16",
                 "TF_ATTENTION_GENERIC", "TF_ATTENTION_MFMA"):
        match = re.search(rf"{name} = (\d+)", text)
        assert match and int(match.group(1)) == getattr(_native, name), name


def test_abi_version_and_variant_selection(lib) -> None:
    assert lib.tf_abi_version() == 15
    variant = lib.tf_paged_gqa_decode_variant
    bf16, f16, f32 = (_native.TF_DTYPE_BFLOAT16, _native.TF_DTYPE_FLOAT16,
                      _native.TF_DTYPE_FLOAT32)
    assert variant(bf16, 64, 8, 16, 0) == _native.TF_ATTENTION_MFMA
    assert variant(f16, 128, 4, 32, 0) == _native.TF_ATTENTION_MFMA
    assert variant(bf16, 32, 16, 16, 0) == _native.TF_ATTENTION_MFMA
    assert variant(f32, 64, 8, 16, 0) == _native.TF_ATTENTION_GENERIC  # fp32: no MFMA path
    assert variant(bf16, 80, 4, 16, 0) == _native.TF_ATTENTION_GENERIC  # head_dim 80
    assert variant(bf16, 64, 32, 16, 0) == _native.TF_ATTENTION_GENERIC  # group > 16
    assert variant(bf16, 64, 8, 4, 0) == _native.TF_ATTENTION_GENERIC  # page of 4 tokens
    assert variant(bf16, 64, 8, 16, _native.TF_ATTENTION_FLAG_FORCE_GENERIC) == 0


def _error(lib) -> str:
    return lib.tf_last_error().decode()


def test_c_abi_rejects_bad_arguments_before_launch(lib) -> None:
    invalid = 1
    stream = None
    fake = 0x1000  # never dereferenced: every call below fails validation first
    status = lib.tf_paged_gqa_decode(
        fake, fake, fake, fake, fake, fake, None, None, None, None, 0, 64,
        2, 8, 3, 64, 4, 16, 8, 256, 1, 0.125, _native.TF_DTYPE_BFLOAT16, 0, stream)
    assert status == invalid and "multiple of kv heads" in _error(lib)
    status = lib.tf_paged_gqa_decode(
        fake, fake, fake, fake, fake, fake, None, None, None, None, 0, 64,
        2, 8, 2, 64, 4, 16, 8, 256, 2, 0.125, _native.TF_DTYPE_BFLOAT16, 0, stream)
    assert status == invalid and "partial buffers" in _error(lib)
    status = lib.tf_paged_gqa_decode(
        fake, fake, fake, fake, fake, fake, fake, fake, fake, None, 3, 64,
        2, 8, 2, 64, 4, 16, 8, 256, 2, 0.125, _native.TF_DTYPE_BFLOAT16, 0, stream)
    assert status == invalid and "too small" in _error(lib)
    status = lib.tf_paged_gqa_decode(
        None, fake, fake, fake, fake, fake, None, None, None, None, 0, 64,
        2, 8, 2, 64, 4, 16, 8, 256, 1, 0.125, _native.TF_DTYPE_BFLOAT16, 0, stream)
    assert status == invalid and "null" in _error(lib)
    status = lib.tf_paged_gqa_decode(
        fake, fake, fake, fake, fake, fake, None, None, None, None, 0, 64,
        2, 8, 2, 64, 4, 16, 8, 256, 1, 0.125, 7, 0, stream)
    assert status == invalid and "dtype" in _error(lib)
    status = lib.tf_rms_norm(fake, fake, fake, 4, 20000, 1e-5, _native.TF_DTYPE_FLOAT16, stream)
    assert status == invalid and "16384" in _error(lib)
    status = lib.tf_rms_norm(fake, fake, fake, 4, 64, 0.0, _native.TF_DTYPE_FLOAT16, stream)
    assert status == invalid and "eps" in _error(lib)
    status = lib.tf_residual_rms_norm(fake, None, fake, fake, fake, 4, 64, 1e-5,
                                      _native.TF_DTYPE_BFLOAT16, stream)
    assert status == invalid and "null" in _error(lib)
    assert lib.tf_swiglu(fake, fake, fake, -1, _native.TF_DTYPE_BFLOAT16, stream) == invalid
    status = lib.tf_paged_kv_write_token(fake, fake, fake, fake, None, None, None, 3, 4, 64,
                                         8, 16, _native.TF_DTYPE_BFLOAT16, stream)
    assert status == invalid and "null" in _error(lib)
    status = lib.tf_paged_kv_write_slots(fake, fake, fake, fake, None, 3, 4, 64, 8, 16,
                                         _native.TF_DTYPE_BFLOAT16, stream)
    assert status == invalid and "slot mapping" in _error(lib)
    status = lib.tf_linear_kstream_norm(fake, 64, fake, 64, fake, 64, 4, 64, 64, 0.0,
                                        _native.TF_DTYPE_BFLOAT16, stream)
    assert status == invalid and "eps" in _error(lib)
    status = lib.tf_linear_kstream_residual(fake, 64, fake, 64, None, 64, fake, 64, 4, 64, 64,
                                            _native.TF_DTYPE_BFLOAT16, stream)
    assert status == invalid and "null" in _error(lib)
    status = lib.tf_linear_kstream_residual(fake, 64, fake, 64, fake, 32, fake, 64, 4, 64, 64,
                                            _native.TF_DTYPE_BFLOAT16, stream)
    assert status == invalid and "residual row stride" in _error(lib)
    status = lib.tf_argmax_rows(fake, 0, 4, 0, _native.TF_DTYPE_BFLOAT16, fake, stream)
    assert status == invalid and "at least one column" in _error(lib)
    status = lib.tf_argmax_rows(fake, 10, 4, 16, _native.TF_DTYPE_BFLOAT16, fake, stream)
    assert status == invalid and "row stride" in _error(lib)
    status = lib.tf_argmax_rows(fake, 16, 4, 16, _native.TF_DTYPE_BFLOAT16, None, stream)
    assert status == invalid and "null" in _error(lib)
    # The message is per call: a successful no-op clears it.
    assert lib.tf_swiglu(fake, fake, fake, 0, _native.TF_DTYPE_BFLOAT16, stream) == 0
    assert _error(lib) == ""


def test_check_maps_status_to_runtime_error(lib) -> None:
    lib.tf_swiglu(None, None, None, 5, 9, None)
    with pytest.raises(RuntimeError, match="swiglu failed .status 1.: unsupported dtype code"):
        _native.check(1, "swiglu")


# ---------------------------------------------------------------------------
# Python mirror: validation order, types and messages of the reference.
# ---------------------------------------------------------------------------
def _cpu_attention_inputs():
    case = make_decode_attention_case([5, 9], query_heads=8, kv_heads=2, head_dim=64,
                                      block_size=16, dtype=torch.float16, seed=0)
    return case.query, case.key_cache, case.value_cache, case.block_tables, case.context_lengths


def test_attention_rejects_cpu_tensors_like_the_reference(lib) -> None:
    """triton_attention.py:341-343: "CUDA" in the message."""

    with pytest.raises(ValueError, match="CUDA"):
        paged_gqa_decode_attention(*_cpu_attention_inputs())


def test_ops_reject_cpu_tensors_like_the_reference(lib) -> None:
    """tests/test_triton_kernels.py:130-140 of the reference."""

    x = torch.randn(2, 64)
    w = torch.ones(64)
    with pytest.raises(ValueError, match="CUDA"):
        rms_norm(x, w)
    with pytest.raises(ValueError, match="CUDA"):
        residual_rms_norm(x, x, w)
    with pytest.raises(ValueError, match="CUDA"):
        swiglu(x, x)
    with pytest.raises(ValueError, match="CUDA"):
        argmax_rows(x)


def test_kv_writes_reject_cpu_tensors(lib) -> None:
    keys = torch.randn(2, 2, 8)
    cache = torch.zeros(4, 4, 2, 8)
    control = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="CUDA"):
        paged_kv_write_token(keys, keys, cache, cache, control, control, control)
    with pytest.raises(ValueError, match="CUDA"):
        paged_kv_write_slots(keys, keys, cache, cache, torch.zeros(2, dtype=torch.int64))
    with pytest.raises(ValueError, match=r"\[batch, kv_heads, head_dim\]"):
        paged_kv_write_token(keys, keys[:1], cache, cache, control, control, control)


def test_autotune_hooks_reject_unknown_operations() -> None:
    """triton_ops.py:263-295: ValueError for an unknown op name."""

    with pytest.raises(ValueError, match="unknown operation"):
        selected_autotune_config("gelu")
    with pytest.raises(ValueError, match="unknown operation"):
        autotune_cache_size("gelu")
    for operation in ("rms_norm", "residual_rms_norm", "swiglu"):
        assert autotune_cache_size(operation) >= 0


def test_norm_launch_shapes_stay_in_the_reference_autotune_set() -> None:
    """The recorded norm launch uses 1, 2, 4 or 8 wavefronts at every width
    (triton_ops.py:28-33) and still holds the row in the register cache
    (8 vectors per lane, 32 scalars)."""

    from tensorforge_amd.kernels.ops import _norm_config

    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        for aligned in (True, False):
            for per_lane in (1, 2):
                for columns in list(range(1, 1100, 7)) + [2048, 4096, 8192, 16383, 16384]:
                    config = _norm_config(columns, dtype, aligned, per_lane)
                    assert config["num_warps"] in {1, 2, 4, 8}, (columns, dtype)
                    width = config["kwargs"]["VECTOR"]
                    capacity = 32 if width == 1 else 8
                    assert config["num_warps"] * 64 * capacity * width >= columns
    assert _norm_config(513, torch.float16, True)["num_warps"] == 8
    assert _norm_config(2048, torch.bfloat16, True)["num_warps"] == 2
    assert _norm_config(4096, torch.bfloat16, True)["num_warps"] == 4


def test_reference_module_paths_resolve_with_the_reference_names() -> None:
    """A caller's `from tensorforge.kernels.<module> import <names>` keeps
    working with only the package prefix changed (the names each reference
    caller imports: runtime/decode_bucket.py:17-22, runtime/batched_decode.py:13,
    runtime/triton_model.py:11, benchmark/attention_benchmark.py:23-27,
    benchmark/kernel_benchmark.py:27-32)."""

    import importlib

    expected = {
        "triton_attention": ("PagedAttentionWorkspace", "is_triton_attention_available",
                             "paged_gqa_decode_attention", "selected_attention_autotune_config"),
        "triton_ops": ("autotune_cache_size", "is_triton_available", "residual_rms_norm",
                       "rms_norm", "selected_autotune_config", "swiglu"),
        "triton_cache": ("paged_kv_write_token",),
    }
    from tensorforge_amd import kernels

    for module_name, names in expected.items():
        module = importlib.import_module(f"tensorforge_amd.kernels.{module_name}")
        for name in names:
            assert callable(getattr(module, name)), (module_name, name)
            public = getattr(kernels, name, None)
            if public is not None:
                assert getattr(module, name) is public, (module_name, name)
    from tensorforge_amd.kernels.triton_attention import is_triton_attention_available
    from tensorforge_amd.kernels.triton_ops import is_triton_available

    assert is_triton_available() is _native.is_available()
    assert is_triton_attention_available() is _native.is_available()


def test_split_size_setting_is_validated_and_restorable() -> None:
    previous = set_attention_split_size(512)
    try:
        assert attention_split_size() == 512
        for bad in (0, -32, 100):
            with pytest.raises(ValueError, match="multiple of 32"):
                set_attention_split_size(bad)
        assert attention_split_size() == 512
        assert set_attention_split_size(None) == 512
        assert attention_split_size() is None
    finally:
        set_attention_split_size(previous)
    assert attention_split_size() == previous


def test_automatic_split_size() -> None:
    """The per-call choice: the reference's 256 for its own split-KV test
    case (1 x 8 heads at 2k, tests/test_decode_attention.py:158-162), 576
    for 72 rows x 4 kv heads at 2k, 2048 for 4 x 8 kv heads at 32k; always
    a multiple of 32 and >= 256."""

    assert attention_split_size_for(2048, 1, 4) == 256
    assert attention_split_size_for(2048, 72, 4) == 576
    assert attention_split_size_for(32768, 4, 8) == 2048
    for context in (1, 17, 300, 4096, 100000):
        for batch in (1, 7, 64, 300):
            size = attention_split_size_for(context, batch, 8)
            assert size >= 256 and size % 32 == 0
            assert -(-context // size) <= max(16, -(-context // 256))


def test_attention_plan() -> None:
    """One pass for wide batches (cfg2: 72 rows x 4 kv heads at 2k, four
    wavefronts per kv head, one per 576 tokens); for narrow calls split-KV
    in partitions of the smallest power of two >= 128 tokens that keeps the
    grid within the compute units (twice that with two kv heads per
    workgroup at D 64) and the workspace's partials, where a row's K and V
    pay for the merge (the reference's own 1 x 8 case with its workspace
    keeps its 256-token partitions), else one pass with up to 4 wavefronts;
    balanced partitions -- up to four kv heads per workgroup, one slot per
    compute unit and group of kv heads, the size set on the device -- for
    2..64 rows of >= 8k when the slots fit one per 256 tokens (cfg3: four
    kv heads per workgroup, 128 slots of >= 256 tokens); two wavefronts per
    split when the caller fixes the partition size or forces split-KV (four
    above 768 tokens), with two kv heads per workgroup for 512-768 tokens."""

    from tensorforge_amd.kernels.attention import (
        balanced_geometry,
        balanced_slots_for,
        narrow_split_plan,
    )

    cfg2 = attention_plan(2048, 72, 4, 2048)
    assert (cfg2.one_pass, cfg2.num_splits, cfg2.waves_per_head) == (True, 1, 4)
    assert cfg2.flags == (9 << 24) | (1 << 20) | (4 << 8)
    short = attention_plan(200, 2, 4, 2048)  # 51 KB of K and V per (row, kv head): one pass
    assert short.one_pass and short.waves_per_head == 4 and short.tokens_per_wave == 64
    assert short.flags == (1 << 24) | (1 << 20) | (4 << 8)
    assert short.split_size == 2048  # the whole table in one partition
    d128 = attention_plan(256, 4, 8, 256, head_dim=128)  # two wavefronts of 128 tokens
    assert d128.one_pass and (d128.waves_per_head, d128.tokens_per_wave) == (2, 128)
    mid16 = attention_plan(1000, 16, 4, 1024)
    assert (mid16.one_pass, mid16.split_size, mid16.num_splits) == (False, 128, 8)
    assert (mid16.heads_per_wg, mid16.waves_per_head) == (2, 2)  # 512 partitions in pairs
    few = attention_plan(2048, 1, 4, 2048)
    assert (few.one_pass, few.split_size, few.num_splits, few.waves_per_head) == (False, 128, 16, 2)
    assert few.flags == (1 << 24) | (1 << 20) | (2 << 8)
    # The reference's 1 x 8 case with its workspace (8 partials per row and head).
    ref = attention_plan(2048, 1, 4, 2048, slot_limit=8)
    assert (ref.one_pass, ref.split_size, ref.num_splits, ref.waves_per_head) == (False, 256, 8, 4)
    assert attention_plan(2048, 48, 4, 2048).one_pass  # 192 workgroups: wide
    narrow32 = attention_plan(2048, 32, 4, 2048)        # 128 workgroups
    assert (narrow32.split_size, narrow32.num_splits, narrow32.heads_per_wg) == (512, 4, 2)
    # Partitions of equal size, about one workgroup per compute unit.
    even = attention_plan(2100, 32, 4, 2112)
    assert (even.split_size, even.num_splits, even.heads_per_wg) == (544, 4, 2)
    assert attention_plan(1000, 32, 4, 1024).one_pass  # 250 KB per (row, kv head), 128 of them
    forty = attention_plan(3000, 40, 4, 3008)  # round(512 / 160) = 3 partitions of pairs
    assert (forty.split_size, forty.num_splits, forty.heads_per_wg) == (1024, 3, 2)
    assert attention_plan(4096, 23, 8, 4096, head_dim=128).one_pass  # 184 workgroups
    long8 = attention_plan(4000, 8, 4, 4096)
    assert (long8.one_pass, long8.split_size, long8.num_splits) == (False, 256, 16)
    d128_8 = attention_plan(1000, 8, 8, 1024, head_dim=128)  # 256-byte slices: no pairs
    assert (d128_8.split_size, d128_8.num_splits, d128_8.heads_per_wg) == (256, 4, 1)
    cfg3 = attention_plan(32768, 4, 8, 32768)
    assert (cfg3.one_pass, cfg3.split_size, cfg3.num_splits, cfg3.balanced) == (False, 256, 128,
                                                                                True)
    assert cfg3.heads_per_wg == 4
    assert cfg3.flags == 32 | (1 << 24) | (4 << 20) | (2 << 8)
    assert balanced_geometry(32768, 4, 8) == (128, 4)
    assert balanced_geometry(16384, 8, 8) == (64, 2)   # 128 slots > 16384 / 256
    assert balanced_geometry(12032, 16, 8) == (32, 1)
    assert balanced_geometry(32768, 4, 4) == (128, 2)  # 256 slots > 32768 / 256
    assert balanced_geometry(32768, 4, 6) == (85, 2)     # 3 groups of 2 kv heads x 85
    assert balanced_geometry(65536, 4, 2) == (256, 2)
    assert balanced_slots_for(32768, 1, 8) == 0      # one row: fixed partitions
    assert balanced_slots_for(8191, 4, 8) == 0       # below 8k
    assert balanced_slots_for(8192, 8, 4) == 0       # 64 slots > 8192 / 256
    assert balanced_slots_for(16384, 8, 4) == 64
    assert balanced_slots_for(16384, 64, 4) == 0     # slots must outnumber rows
    assert balanced_slots_for(65536, 65, 1) == 0     # at most 64 rows
    assert not attention_plan(8192, 8, 4, 8192).balanced
    one_row = narrow_split_plan(32768, 1, 4, 64, 2)
    assert (one_row.split_size, one_row.num_splits, one_row.heads_per_wg) == (256, 128, 2)
    assert narrow_split_plan(32768, 1, 4, 64, 2, slot_limit=64).split_size == 512
    assert narrow_split_plan(4000, 1, 4, 64, 2).split_size == 128
    assert narrow_split_plan(4000, 1, 4, 64, 2, slot_limit=0) is None
    assert narrow_split_plan(512, 4, 4, 64, 2) is None  # 128 KB per (row, kv head)
    assert narrow_split_plan(512, 4, 8, 128, 2) is not None  # 256 KB
    assert attention_plan(4096, 64, 4, 4096).waves_per_head == 8
    mid = attention_plan(1024, 64, 4, 1024)  # ~4 wavefronts per row below 1.5k
    assert (mid.waves_per_head, mid.tokens_per_wave) == (4, 256)
    assert attention_plan(512, 64, 4, 512).tokens_per_wave == 128
    assert attention_plan(100, 64, 4, 128).flags == 0  # one wavefront
    assert attention_plan(32768, 64, 4, 32768).waves_per_head == 8
    forced = attention_plan(2048, 72, 4, 2048, "split_kv")
    assert (forced.one_pass, forced.split_size, forced.waves_per_head) == (False, 576, 2)
    assert forced.heads_per_wg == 2
    assert forced.tokens_per_wave == 0  # every wavefront streams its share of the partition
    previous = set_attention_split_size(512)
    try:
        fixed = attention_plan(2048, 72, 4, 2048)
        assert (fixed.one_pass, fixed.split_size, fixed.num_splits) == (False, 512, 4)
        # 512-768-token partitions: two kv heads per workgroup
        assert fixed.flags == ((2 << _native.TF_ATTENTION_HEADS_PER_WG_SHIFT)
                               | (2 << _native.TF_ATTENTION_WAVES_PER_CU_SHIFT))
        set_attention_split_size(256)
        assert attention_plan(2048, 72, 4, 2048).heads_per_wg == 1
        assert attention_plan(2048, 72, 3, 2048).heads_per_wg == 1  # odd kv heads
        set_attention_split_size(512)
        assert attention_plan(400, 2, 4, 2048).waves_per_head == 1  # one pass
        set_attention_split_size(1024)
        assert attention_plan(32768, 4, 8, 32768).waves_per_head == 4
    finally:
        set_attention_split_size(previous)


def test_workspace_capacity_contract() -> None:
    """triton_attention.py:25-57: programs = B * Hq * ceil(ctx / 256) fp32
    rows, accumulator rows padded to next_pow2(head_dim)."""

    workspace = PagedAttentionWorkspace.allocate(
        batch_capacity=3, query_heads=8, head_dim=80, max_context_length=1000,
        device=torch.device("cpu"),
    )
    programs = 3 * 8 * 4
    assert workspace.partial_max.shape == (programs,)
    assert workspace.partial_sum.shape == (programs,)
    assert workspace.partial_accumulator.shape == (programs, 128)
    assert workspace.partial_max.dtype == torch.float32
    assert workspace.split_counters is not None
    assert workspace.split_counters.dtype == torch.int32
    assert not bool(workspace.split_counters.any())
    with pytest.raises(ValueError, match="positive"):
        PagedAttentionWorkspace.allocate(batch_capacity=0, query_heads=8, head_dim=64,
                                         max_context_length=16, device=torch.device("cpu"))
    # Frozen: the fields of a workspace captured in a graph cannot be rebound.
    with pytest.raises(AttributeError):
        workspace.partial_max = torch.empty(1)  # type: ignore[misc]
    # The three reference fields alone still form a workspace.
    bare = PagedAttentionWorkspace(workspace.partial_max, workspace.partial_sum,
                                   workspace.partial_accumulator)
    assert bare.split_counters is None


# ---------------------------------------------------------------------------
# Workloads and byte models.
# ---------------------------------------------------------------------------
def test_decode_attention_byte_model_matches_reference_formula() -> None:
    """attention_benchmark.py:148-161 for a single-length batch:
    (2 q + 2 kv) elements * e + B * (ceil(ctx / page) + 1) * 4."""

    batch, hq, hkv, d, ctx, page, e = 4, 32, 8, 128, 1000, 16, 2
    q_elements = batch * hq * d
    kv_elements = batch * ctx * hkv * d
    expected = (2 * q_elements + 2 * kv_elements) * e + batch * ((ctx + page - 1) // page + 1) * 4
    assert decode_attention_bytes([ctx] * batch, hq, hkv, d, page, e) == expected
    assert decode_attention_bytes([0, ctx], hq, hkv, d, page, e) == expected // batch


def test_config2_workload_is_the_documented_one() -> None:
    lengths = tinyllama_decode_lengths(0)
    assert len(lengths) == 72 and lengths[64:] == [0] * 8
    assert all(128 <= ctx <= 2048 for ctx in lengths[:64])
    case = tinyllama_decode_case(0)
    assert tuple(case.query.shape) == (72, 32, 64)
    assert case.key_cache.shape[1:] == (16, 4, 64)
    assert case.query.dtype == torch.bfloat16
    assert sum(case.lengths) == 77431
    assert decode_attention_bytes(case.lengths, 32, 4, 64, 16, 2) == 79833372


def test_elementwise_byte_models() -> None:
    assert rms_norm_bytes(8, 2048, 2, residual=False) == (2 * 8 + 1) * 2048 * 2
    assert rms_norm_bytes(8, 2048, 2, residual=True) == (4 * 8 + 1) * 2048 * 2
    assert swiglu_bytes(5632, 2) == 3 * 5632 * 2
    assert kv_append_bytes(64, 4, 64, 2) > 0


def test_decode_step_byte_model_closed_form() -> None:
    """TinyLlama geometry: 44,040,192 weight elements per layer plus two
    2048-element gains (qkv 2560 x 2048, o 2048 x 2048, gate|up 11264 x
    2048, down 2048 x 5632), 22 layers, 1.94 GB in bf16; K/V 512 bytes per
    token and layer for each of K and V."""

    from tensorforge_amd.decode import tinyllama_config
    from tensorforge_amd.workloads import decode_step_bytes

    config = tinyllama_config()
    parts = decode_step_bytes(config, sum_context=1000, batch=2, element_size=2)
    assert parts["layer_weights"] == 22 * (44_040_192 + 2 * 2048) * 2
    assert parts["kv_read"] == 22 * 1000 * 4 * 64 * 2 * 2
    assert parts["kv_write"] == 22 * 2 * 4 * 64 * 2 * 2
    assert parts["lm_head"] == (32000 * 2048 + 2048) * 2
    assert parts["embedding_and_logits"] == 2 * 2048 * 2 + 2 * 32000 * 2
    assert parts["total"] == sum(v for key, v in parts.items() if key != "total")
    assert abs(parts["layer_weights"] / 1e9 - 1.938) < 0.001


def test_bench_refuses_more_than_one_gpu() -> None:
    result = subprocess.run(
        [sys.executable, str(REPO_ROOT / "bench.py"), "--gpus", "2"],
        capture_output=True, text=True, timeout=300,
    )
    assert result.returncode == 2
    message = json.loads(result.stdout.strip().splitlines()[-1])
    assert "one GPU" in message["error"] and message["n_gpus"] == 2


def test_noalloc_attention_rejects_what_its_scratch_cannot_hold(lib) -> None:
    """The size checks of tf_paged_gqa_decode_noalloc come before any HIP
    call: 4 rows x 32 heads x 2048 splits of (64 + 2) floats exceed the
    8 MiB array, and flag bits with no meaning in this ABI (bit 2 once
    selected a streaming kernel that has been removed) are rejected."""

    bf16 = _native.TF_DTYPE_BFLOAT16
    call = lib.tf_paged_gqa_decode_noalloc
    status = call(None, None, None, None, None, None, 4, 32, 4, 64, 10, 16, 64, 32, 2048,
                  0.125, bf16, 0, None)
    assert status == 1 and b"no-allocation scratch holds 8388608" in lib.tf_last_error()
    for bits in (4, 8, 2 << 16):
        status = call(None, None, None, None, None, None, 4, 32, 4, 64, 10, 16, 64, 32, 2, 0.125,
                      bf16, bits, None)
        assert status == 2 and b"unknown attention flag bits" in lib.tf_last_error()
    assert _native.TF_NOALLOC_SCRATCH_BYTES == 8 << 20


def test_measurement_probes_reject_bad_arguments_before_launch(lib) -> None:
    """The read and page-gather probes validate sizes, shapes and pointers on
    the host: nothing reaches the device (no GPU here)."""

    sink = ctypes.c_uint32(0)
    read = lib.tf_hbm_read_probe
    assert read(None, 1 << 20, 256, 4, 4, ctypes.byref(sink), None) == 1          # no buffer
    assert read(ctypes.c_void_p(16), 100, 256, 4, 4, ctypes.byref(sink), None) == 1  # not x16
    assert read(ctypes.c_void_p(16), 1 << 20, 256, 17, 4, ctypes.byref(sink), None) == 1
    gather = lib.tf_hbm_page_gather_probe
    page = ctypes.c_void_p(256)
    assert gather(page, page, page, 10, 1000, 64, 256, 8, ctypes.byref(sink), None) == 1  # % 1024
    assert gather(page, page, page, 10, 8192, 0, 256, 8, ctypes.byref(sink), None) == 1   # blocks
    assert gather(page, page, None, 10, 8192, 64, 256, 8, ctypes.byref(sink), None) == 1  # list
    assert gather(page, ctypes.c_void_p(8), page, 10, 8192, 64, 256, 8, ctypes.byref(sink),
                  None) == 1                                                           # aligned
    assert b"page gather probe" in lib.tf_last_error()
    # an empty page list is a no-op that launches nothing
    assert gather(None, None, None, 0, 8192, 64, 256, 8, ctypes.byref(sink), None) == 0
