"""CPU checks of the C-ABI library: it loads, exports every entry point that
include/opure_hip.h declares, and its host-only helpers and error paths behave
(no kernel is launched here)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import opure_hip as H
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "opure_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(opure_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = H.lib()
    names = declared_symbols()
    assert len(names) >= 35
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_binding_declares_every_symbol():
    L = H.lib()
    for n in declared_symbols():
        assert getattr(L, n).argtypes is not None, n


@pytest.mark.parametrize("mode", [H.ROPE_GPU, H.ROPE_CPUREF])
def test_rope_table_matches_oracle(mode):
    a = H.rope_table(500000.0, 128, 1024, mode)
    b = O.rope_table(500000.0, 128, 1024, mode)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_error_paths_without_device():
    L = H.lib()
    assert L.opure_rope_table(10000.0, 3, 4, 0, None, None) == H.E_INVALID
    assert b"bad argument" in L.opure_last_error()
    assert L.opure_dev_create(0, None) == H.E_INVALID
    assert L.opure_gemv_batched_f32(None, None) == H.E_INVALID
    assert L.opure_verify_step(None, None) == H.E_INVALID
    assert L.opure_verify_layer(None, None) == H.E_INVALID
    assert L.opure_kv_rollback(None, None) == H.E_INVALID
    assert L.opure_graph_destroy(None) == H.OK


STRUCTS = {
    "opure_linear": H.Linear, "opure_layer_weights": H.LayerWeights, "opure_model": H.Model,
    "opure_kv": H.KV, "opure_gemv_args": H.GemvArgs, "opure_attn_args": H.AttnArgs,
    "opure_accept_args": H.AcceptArgs, "opure_sample_args": H.SampleArgs,
    "opure_rollback_args": H.RollbackArgs, "opure_verify_args": H.VerifyArgs,
    "opure_verify_layer_args": H.VerifyLayerArgs,
}


def test_struct_layouts_match_header(tmp_path):
    """Compile a probe against include/opure_hip.h and compare every struct's
    size and field offsets with the ctypes mirror."""
    import subprocess
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "opure_hip.h"', "int main(void){"]
    for cname, cls in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            cf = "in" if fname == "in_" else fname
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {cf}));')
    lines.append("return 0;}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = {}
    for ln in out:
        if ln.strip():
            a, b, c = ln.split()
            got[(a, b)] = int(c)
    for cname, cls in STRUCTS.items():
        assert got[(cname, "size")] == C.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert got[(cname, fname)] == getattr(cls, fname).offset, (cname, fname)


# ---- the native engine (include/opure_engine.h, libopure_engine.so) -------
def engine_symbols():
    text = open(os.path.join(ROOT, "include", "opure_engine.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|const char\s*\*)\s+(opure_[a-z0-9_]+)\s*\(", text, flags=re.M)))


def test_engine_library_exports_every_declared_symbol():
    import opure_engine as E
    L = E.lib()
    names = engine_symbols()
    assert len(names) >= 25 and "opure_model_load" in names and "opure_page_pool_grow_seq" in names
    assert not [n for n in names if not hasattr(L, n)]


def test_engine_struct_layouts_match_header(tmp_path):
    import subprocess
    import opure_engine as E
    structs = {"opure_engine_options": E.Options, "opure_engine_stats": E.Stats, "opure_engine_metrics": E.Metrics,
               "opure_load_options": E.LoadOptions, "opure_model_info": E.ModelInfo,
               "opure_host_linear": E.HostLinearC, "opure_tensor_info": E.TensorInfo}
    cname_of = {"in_": "in"}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "opure_engine.h"', "int main(void){"]
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {cname_of.get(fname, fname)}));')
    lines.append("return 0;}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    for ln in out:
        if not ln:
            continue
        cname, field, val = ln.split()
        cls = structs[cname]
        want = C.sizeof(cls) if field == "size" else getattr(cls, field).offset
        assert int(val) == want, (cname, field, val, want)


def test_engine_error_paths_without_device():
    import opure_engine as E
    L = E.lib()
    h = C.c_void_p()
    assert L.opure_engine_create(None, None, None, None, C.byref(h)) == H.E_INVALID
    assert b"null argument" in L.opure_engine_last_error()
    assert L.opure_engine_generate(None, None, 0, 0, None, None) == H.E_INVALID
    assert L.opure_engine_generate_speculative(None, None, 0, 0, None, None, 0, None) == H.E_INVALID
    assert L.opure_engine_destroy(None) == H.OK
    assert L.opure_model_files_open(None, None, C.byref(h)) == H.E_INVALID
    assert L.opure_model_load(None, b"/nonexistent", None, C.byref(h)) == H.E_INVALID
    assert L.opure_engine_initialize(None, None, None, None, None, C.byref(h)) == H.E_INVALID
    assert L.opure_safetensors_open(b"/nonexistent/model.safetensors", C.byref(h)) == H.E_INVALID
    assert b"cannot open" in L.opure_engine_last_error()
    assert L.opure_model_files_open(b"/nonexistent", None, C.byref(h)) == H.E_INVALID
    assert b"config.json" in L.opure_engine_last_error()


def test_empty_page_pool_is_refused_before_any_launch():
    """A cache with no pages (n_pages = 0 or no page-table columns) is refused
    by attention, rollback and (through attention's check) the verify step,
    before anything touches the device: the folded attention kernel reads
    page 0 for a missing entry, so a pool must hold one page.  The device
    handle below is a placeholder the calls never dereference."""
    L = H.lib()
    fake = C.create_string_buffer(256)                      # stands in for device pointers and the handle
    addr = C.addressof(fake)
    m = H.Model()
    m.n_layers, m.hidden, m.n_heads, m.n_kv_heads, m.head_dim = 1, 256, 4, 2, 64
    m.ffn, m.vocab, m.afmt, m.wfmt = 512, 1024, H.A_F16, H.W_I8PC
    for n_pages, max_pages in ((0, 4), (4, 0)):
        kv = H.KV(addr, n_pages, H.PAGE_SIZE, addr, max_pages)
        a = H.AttnArgs(C.pointer(m), C.pointer(kv), 0, 1, 4, addr, 16, addr, addr)
        assert L.opure_attn_decode_paged(addr, C.byref(a)) == H.E_INVALID
        assert b"no pages" in L.opure_last_error()
        rb = H.RollbackArgs(C.pointer(m), C.pointer(kv), 1, 3, addr, addr, addr, None, 0, None, 0, 0)
        assert L.opure_kv_rollback(addr, C.byref(rb)) == H.E_INVALID
        assert b"no pages" in L.opure_last_error()
