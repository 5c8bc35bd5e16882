"""CPU: the C-ABI library loads and exports every entry point include/*.h declares,
and the ctypes signature table covers exactly those entry points."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kessie_mi355x.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n.startswith(("kessie_", "launch_kessie_"))))


def test_header_declares_the_reference_launchers():
    names = declared_functions()
    for ref in ("launch_kessie_windowed_attn", "launch_kessie_fused_fog_attn", "launch_kessie_page_evict",
                "launch_kessie_page_insert", "launch_kessie_rope_remap"):
        assert ref in names


def test_library_exports_every_declared_symbol():
    from kessie_amd import _lib

    path = None
    for cand in _lib.candidates():
        if os.path.exists(cand):
            path = cand
            break
    if path is None:
        pytest.fail("libkessie_mi355x.so is not built (run python -m kessie_amd.build)")
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    exported = set(ln.split()[-1] for ln in out.splitlines() if ln.strip())
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    # Host-side helpers stay hidden (HIP itself exports the kernels' host stubs).
    leaked = [n for n in exported if n.startswith("_ZN6kessie") and "kernel" not in n]
    assert not leaked, f"internal symbols exported: {leaked[:5]}"


def declared_arity():
    """name -> number of parameters, parsed from the header's declarations."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b((?:launch_)?kessie_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_signature_table_matches_header():
    from kessie_amd import _lib

    assert sorted(_lib.SIGNATURES) == declared_functions()
    arity = declared_arity()
    assert sorted(arity) == declared_functions()
    for name, (_, args) in _lib.SIGNATURES.items():
        assert len(args) == arity[name], f"{name}: ctypes has {len(args)} args, header {arity[name]}"


def test_loads_and_reports_errors_without_gpu():
    """Host-side argument validation runs before any HIP call, so it works here."""
    from kessie_amd import _lib

    lib = _lib.load()
    assert lib.kessie_version() >= 100
    st = lib.kessie_rope_remap_paged(None, 0, 0, 0, None, 0, None, None, None, 4, 8, 128, 16, 1, None)
    assert st == _lib.ERR_INVALID
    status, msg = _lib.last_error()
    assert status == _lib.ERR_INVALID and "inv_freq" in msg
    st = lib.kessie_page_select_evict(None, None, 10, -1, 0.25, None, None, None, 0, None)
    assert st == _lib.ERR_INVALID
    # Workspace sizing is a pure host computation.
    assert lib.kessie_fog_decode_workspace_bytes(16, 32, 8, 128, 131072, 16, 1) > 0
    assert lib.kessie_page_workspace_bytes(65536) >= 65536 * 4


def test_decode_splits_counted_in_16_token_blocks():
    """The decode's split count (and so its workspace) is taken in 16-token
    blocks, so pages of 32 or 64 tokens split a context as 16-token pages do;
    smaller pages count as they are.  Host computation (the CU count falls back
    to 256 without a device)."""
    from kessie_amd import _lib

    lib = _lib.load()
    for b, ctx in [(1, 4096), (1, 16384), (16, 131072), (3, 1000)]:
        s16 = lib.kessie_fog_decode_num_splits(b, 8, ctx, 16)
        assert lib.kessie_fog_decode_num_splits(b, 8, ctx, 32) == s16
        assert lib.kessie_fog_decode_num_splits(b, 8, ctx, 64) == s16
        assert (lib.kessie_fog_decode_workspace_bytes(b, 32, 8, 128, ctx, 32, 1)
                == lib.kessie_fog_decode_workspace_bytes(b, 32, 8, 128, ctx, 16, 1))
    assert lib.kessie_fog_decode_num_splits(1, 8, 64, 8) == 4  # 8 pages of 8 tokens: at least 2 per split


def test_ctypes_class_mirrors_reference_surface():
    from kessie_amd.kessie_hip_ctypes import KeSSieKernels

    for name in ("windowed_attention", "fused_fog_attention", "rope_remap", "page_evict", "page_insert",
                 "create_stream", "sync_stream", "_get_stream_ptr", "_ptr"):
        assert callable(getattr(KeSSieKernels, name))


def test_prefill_and_decode_argument_errors_without_gpu():
    """The paged entry points reject bad arguments before any launch: missing
    query_start_loc / page table (invalid), a shape the MFMA varlen kernel does
    not take (unsupported), a split prefill without room for its partials
    (workspace).  Fake 16-byte-aligned addresses stand in for device buffers:
    none of these paths reads them."""
    import ctypes as C

    from kessie_amd import _lib

    lib = _lib.load()
    fake = C.c_void_p(1 << 20)
    bf16 = _lib.DTYPE_BF16
    # varlen: query_start_loc missing
    st = lib.kessie_fog_prefill_varlen(fake, None, 64, fake, 1024, 65536, 4096, 2048, 128, fake, 64, fake,
                                       None, 0, None, 0, fake, 2, 32, 8, 128, 16, 1024, 0, 0.088, 1, bf16,
                                       None, 0, None)
    assert st == _lib.ERR_INVALID
    # varlen: head_dim 64 is not an MFMA shape
    st = lib.kessie_fog_prefill_varlen(fake, fake, 64, fake, 1024, 32768, 2048, 1024, 64, fake, 64, fake,
                                       None, 0, None, 0, fake, 2, 32, 8, 64, 16, 1024, 0, 0.125, 1, bf16,
                                       None, 0, None)
    assert st == _lib.ERR_UNSUPPORTED
    # paged prefill: a 64-query chunk on 64K keys splits the key range and needs a workspace
    need = lib.kessie_fog_prefill_workspace_bytes(1, 64, 32, 8, 128, 65536, 16, bf16)
    assert need > 0
    st = lib.kessie_fog_prefill_paged(fake, fake, 4096, 65536, 4096, 2048, 128, fake, 4096, fake, None, 0,
                                      None, 0, fake, 1, 64, 32, 8, 128, 16, 65536, 0, 0.088, 1, bf16,
                                      None, 0, None)
    assert st == _lib.ERR_WORKSPACE
    status, msg = _lib.last_error()
    assert status == _lib.ERR_WORKSPACE and "workspace" in msg
    # decode: page table missing
    st = lib.kessie_fog_decode_paged(fake, fake, 4096, 65536, 4096, 2048, 128, None, 4096, fake, None, 0,
                                     None, 0, fake, 1, 32, 8, 128, 16, 4096, 0, 0.088, bf16, None, 0, None)
    assert st == _lib.ERR_INVALID
    # score eviction: every byte offset of its range-limited loads must stay below 2^31
    st = lib.kessie_page_select_evict(fake, fake, 1 << 29, -1, 0.25, fake, fake, fake, 1 << 40, None)
    assert st == _lib.ERR_UNSUPPORTED
    other = C.c_void_p(1 << 21)  # new_tables must differ from tables
    st = lib.kessie_page_evict_compact(fake, fake, 4096, -1, 0.25, fake, fake, fake, fake, 1, 1 << 29, other, fake,
                                       fake, fake, fake, 1 << 40, None)
    assert st == _lib.ERR_UNSUPPORTED
    status, msg = _lib.last_error()
    assert status == _lib.ERR_UNSUPPORTED and "2^29" in msg


PROBES_HEADER = os.path.join(ROOT, "include", "kessie_probes.h")


def test_probe_library_is_separate_from_the_product():
    """The measurement probes live in their own library: declared in
    kessie_probes.h, exported by libkessie_probes.so, absent from the product."""
    from kessie_amd import build as kbuild

    text = re.sub(r"/\*.*?\*/", "", open(PROBES_HEADER).read(), flags=re.S)
    probes = sorted(set(re.findall(r"\b(kessie_probe_[a-z0-9_]+)\s*\(", text)))
    assert probes == ["kessie_probe_copy", "kessie_probe_page_rows", "kessie_probe_stream_read"]
    for path, want in ((kbuild.PROBES_LIB_PATH, True), (kbuild.LIB_PATH, False)):
        if not os.path.exists(path):
            pytest.fail(f"{path} is not built (run python -m kessie_amd.build)")
        out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                             check=True).stdout
        exported = set(ln.split()[-1] for ln in out.splitlines() if ln.strip())
        for name in probes:
            assert (name in exported) == want, (path, name)
    assert not any(n.startswith("kessie_probe") for n in declared_functions())
