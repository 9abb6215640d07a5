"""CPU checks of the C ABI: the library loads and exports every declared entry
point, and argument errors are reported without touching a GPU."""

from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

import pytest
import torch  # noqa: F401  (loads the HIP runtime the library binds to)

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))
LIB_PATH = Path(os.environ.get("FRWKV_TEST_LIBRARY")
                or ROOT / "flashrwkv_amd" / "libflashrwkv_amd.so")

DECL = re.compile(r"^[A-Za-z_][\w\s\*]*?\b(frwkv_\w+)\s*\(", re.MULTILINE)


def declared_symbols() -> list[str]:
    names = []
    for header in HEADERS:
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.DOTALL)
        names.extend(DECL.findall(text))
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not LIB_PATH.exists():
        pytest.fail(f"{LIB_PATH} is not built; run python -m flashrwkv_amd._build")
    return ctypes.CDLL(str(LIB_PATH))


def test_header_declares_entry_points():
    names = declared_symbols()
    for required in ("frwkv_abi_version", "frwkv_status_string", "frwkv_last_error",
                     "frwkv_metadata_validate", "frwkv_recurrent_forward"):
        assert required in names


def test_every_declared_symbol_is_exported(lib):
    missing = [name for name in declared_symbols() if not hasattr(lib, name)]
    assert not missing, missing


def test_version_and_status_strings(lib):
    lib.frwkv_abi_version.restype = ctypes.c_int
    header = (ROOT / "include" / "flashrwkv_amd.h").read_text()
    version = int(re.search(r"#define FRWKV_ABI_VERSION (\d+)", header).group(1))
    assert lib.frwkv_abi_version() == version
    lib.frwkv_status_string.restype = ctypes.c_char_p
    assert lib.frwkv_status_string(0) == b"ok"
    assert lib.frwkv_status_string(1) == b"invalid argument"
    assert lib.frwkv_status_string(99) == b"unknown status"


def test_null_pointers_are_rejected_before_any_launch(lib):
    lib.frwkv_last_error.restype = ctypes.c_char_p
    null = ctypes.c_void_p()
    rc = lib.frwkv_metadata_validate(null, null, 1, 1, 1, null, null, null, null)
    assert rc == 1
    assert b"null pointer" in lib.frwkv_last_error()
    args = [ctypes.c_int(2), ctypes.c_int(0)] + [ctypes.c_int32(1)] * 6 + [null] * 12 \
        + [ctypes.c_float(1.0), null]
    assert lib.frwkv_recurrent_forward(*args) == 1
    assert b"null pointer" in lib.frwkv_last_error()


def _header_parameter_counts() -> dict[str, int]:
    text = (ROOT / "include" / "flashrwkv_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.DOTALL)
    counts = {}
    for match in re.finditer(r"\b(frwkv_\w+)\s*\(([^)]*)\)\s*;", text):
        params = match.group(2).strip()
        counts[match.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return counts


def test_ctypes_binding_matches_header_signatures():
    """flashrwkv_amd.capi (the binding the GPU boundary tests use) declares
    every entry point with the header's parameter count."""
    from flashrwkv_amd import capi

    counts = _header_parameter_counts()
    assert set(counts) == set(capi.SIGNATURES)
    for name, argtypes in capi.SIGNATURES.items():
        assert len(argtypes) == counts[name], name


def test_ctypes_binding_reports_errors_without_a_gpu():
    from flashrwkv_amd import capi

    lib = capi.library()
    null = ctypes.c_void_p()
    rc = lib.frwkv_chunk_forward(2, 1, 0, 1, 1, 64, 1, 1, *([null] * 12), 1.0, null)
    assert rc == 1 and b"null pointer" in lib.frwkv_last_error()
    with pytest.raises(RuntimeError, match="invalid argument"):
        capi._check(rc)


def test_fp16_state_entry_points_reject_bad_arguments_without_a_gpu():
    from flashrwkv_amd import capi

    lib = capi.library()
    null = ctypes.c_void_p()
    rc = lib.frwkv_recurrent_fp16_forward(1, 1, 64, 1, 1, 1, *([null] * 13), 1.0, null)
    assert rc == 1 and b"null pointer" in lib.frwkv_last_error()
    assert lib.frwkv_advance_i32(null, 0, 5, null) == 1
    assert b"non-empty" in lib.frwkv_last_error()
    assert lib.frwkv_advance_i32_varlen(1, 4, null, null, null, null, null) == 1
    # Odd row length: rejected before any pointer is touched.
    fake = ctypes.c_void_p(0x1000)
    assert lib.frwkv_add_vec(3, 7, fake, fake, fake, null) == 1
    assert b"even C" in lib.frwkv_last_error()


DIRECT_ENTRY_POINTS = (
    "recurrent_fp32_from_decay_logits", "recurrent_fp32_forward_internal",
    "recurrent_fp16_from_decay_logits", "recurrent_fp16_advance_i32",
    "recurrent_fp16_advance_i32_varlen", "recurrent_add_vec_forward_varlen",
    "tmix_kk_a_gate_forward_varlen", "tmix_lnx_rkvres_xg_forward_varlen",
    "recurrent_tmix_fused_forward",
)


def test_direct_entry_points_match_the_ops_without_a_gpu():
    """The pybind11 entry points of the decode chain exist, and an argument
    error reads exactly as it does through the TORCH_LIBRARY op (no backtrace),
    raised before anything reaches a GPU (CPU tensors are rejected first)."""
    from flashrwkv_amd import _C

    for name in DIRECT_ENTRY_POINTS:
        assert callable(getattr(_C.direct, name)), name
        assert hasattr(_C.ops, name), name
    tok = [torch.zeros(1, 1, 64, dtype=torch.bfloat16) for _ in range(7)]
    args = (torch.tensor([0, 1], dtype=torch.int32), torch.zeros(1, dtype=torch.int32),
            torch.zeros(1, 1, 64, 64), *tok, 1.0, None, None, -1)
    with pytest.raises(RuntimeError) as via_op:
        _C.ops.recurrent_fp32_from_decay_logits(*args)
    with pytest.raises(RuntimeError) as via_direct:
        _C.direct.recurrent_fp32_from_decay_logits(*args)
    assert str(via_direct.value) == str(via_op.value)
    assert "must be CUDA" in str(via_direct.value)
    assert "Exception raised from" not in str(via_direct.value)
    # A metadata argument that is not a ticket is named in the error.
    with pytest.raises(RuntimeError, match="validated_metadata must be None or a ticket"):
        _C.direct.recurrent_fp32_from_decay_logits(*args[:12], "not a ticket", -1)
    # The public facade goes through the direct entry point.
    with pytest.raises(RuntimeError, match="must be CUDA"):
        _C.recurrent_fp32_from_decay_logits(*args[:10], 1.0)


def test_library_imports_no_allocating_or_synchronizing_hip_call():
    """The library's only HIP imports are kernel registration, launch and
    error queries: no entry point allocates or frees device memory, copies,
    sets memory or waits on the host (callers bring every buffer)."""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm is not installed")
    out = subprocess.run([nm, "-D", "--undefined-only", str(LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    imported = {line.split()[-1].split("@")[0] for line in out.splitlines()
                if "hip" in line.lower()}
    allowed = {"__hipPopCallConfiguration", "__hipPushCallConfiguration",
               "__hipRegisterFatBinary", "__hipRegisterFunction", "__hipUnregisterFatBinary",
               "__hipRegisterVar", "__hipRegisterManagedVar", "hipGetErrorString",
               "hipGetLastError", "hipLaunchKernel",
               # the static scratch of the allocation-free backward variant
               "hipGetDevice", "hipGetSymbolAddress"}
    assert imported <= allowed, sorted(imported - allowed)
    assert "hipLaunchKernel" in imported


@pytest.mark.parametrize("head_size,piece,elem", [(64, 64, 4), (128, 16, 2), (256, 16, 4)])
def test_interior_bytes_per_head_size(head_size, piece, elem):
    """The interior-state buffer holds ceil(N / P) slots of H x D x D states:
    fp32 at head sizes 64 and 256, bf16 at 128 (the piece kernels' layout);
    a backward without it needs that much workspace beside its slices."""
    from flashrwkv_amd import capi

    for heads, n_tok in ((1, 1), (3, 130), (32, 4096)):
        want = -(-n_tok // piece) * heads * head_size * head_size * elem
        assert capi.statetune_interior_bytes(head_size, heads, n_tok) == want
        assert (capi.statetune_backward_workspace_bytes(head_size, heads, n_tok, False)
                - capi.statetune_backward_workspace_bytes(head_size, heads, n_tok, True)) == want
    assert capi.statetune_interior_bytes(head_size, 0, 16) == 0


def test_noalloc_backward_rejects_oversized_need_without_a_gpu():
    """frwkv_statetune_backward_noalloc compares the workspace it needs with
    its static scratch before anything else: head size 256 with 4096 tokens
    is refused with an argument error (the placeholder pointers are never
    used)."""
    from flashrwkv_amd import capi

    lib = capi.library()
    fake = ctypes.c_void_p(256)
    need = capi.statetune_backward_workspace_bytes(256, 1, 4096, False)
    assert need > capi.NOALLOC_SCRATCH_BYTES
    rc = lib.frwkv_statetune_backward_noalloc(2, 1, 1, 1, 256, 4096, 1, *([fake] * 21), 1.0,
                                              None)
    assert rc == 1 and b"bytes of scratch" in lib.frwkv_last_error()


def test_chunk_forward_rejects_too_many_heads_without_a_gpu(lib):
    """The chunked kernels' 32-bit row offsets bound the head count (65536);
    a larger one is refused before any launch."""
    lib.frwkv_last_error.restype = ctypes.c_char_p
    fake = ctypes.c_void_p(256)  # never dereferenced: the call fails first
    null = ctypes.c_void_p()
    i32 = ctypes.c_int32
    common = [i32(1), i32(1 << 17), i32(64), i32(64), i32(1)]
    ptrs = [fake] * 4 + [fake, fake, null, fake, fake, fake, fake, fake]
    rc = lib.frwkv_chunk_forward(ctypes.c_int(2), ctypes.c_int(1), ctypes.c_int(0), *common,
                                 *ptrs, ctypes.c_float(1.0), null)
    assert rc == 2
    assert b"at most 65536 heads" in lib.frwkv_last_error()


def test_backward_without_interior_or_workspace_is_refused_without_a_gpu():
    """frwkv_statetune_backward at head size 64 with neither the forward's
    interior states nor a workspace is an argument error before any launch:
    whether a chunk spans more than one 64-token piece is only known on the
    device, and such a chunk needs the recomputed interior states (a 100-token
    chunk here; the placeholder pointers are never used)."""
    from flashrwkv_amd import capi

    lib = capi.library()
    fake = ctypes.c_void_p(256)
    null = ctypes.c_void_p()
    # io bf16, raw decay, B=1, H=1, D=64, N=100, one chunk.
    head = [2, 1, 1, 1, 64, 100, 1]
    metadata_and_boundary = [fake] * 4           # offsets, starts, ends, boundary
    tensors = [fake, fake, null, fake, fake, fake, fake, fake, fake]  # r..b, dy, dS_T
    grads = [fake] * 7
    rc = lib.frwkv_statetune_backward(*head, *metadata_and_boundary, null, *tensors[:2],
                                      *tensors[2:], *grads, null, 0, 1.0, None)
    assert rc == 1
    assert b"workspace of 0 bytes given" in lib.frwkv_last_error()
