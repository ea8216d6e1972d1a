"""The C ABI: every function include/*.h declares is exported by the library
that provides it (libtgrt.so for tgrt.h, each generated variant library for
tilegen_launch.h), and the libraries load without a GPU.  No compute calls."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import pytest

from tilegen_amd import runtime
from tilegen_amd.codegen import Config, generate
from tilegen_amd.dsl import standard_kernels
from tilegen_amd.verify import compile_generated

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header: str):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tg_[a-z_0-9]+|tgv_[a-z_0-9]+|launch_[a-z_0-9]+)\s*\(",
                                 text)))


def _exported(path: str):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_runtime_exports_every_declared_symbol():
    declared = _declared("tgrt.h")
    assert len(declared) >= 25
    exported = _exported(runtime.lib_path())
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    L = runtime.lib()  # loads without a GPU
    for s in declared:
        assert hasattr(L, s)


@pytest.mark.parametrize("kernel", ["spmv", "spmm", "sddmm", "fused_spmv_axpy", "axpy"])
def test_variant_library_exports_launch_abi(kernel, tmp_path):
    gen = generate(standard_kernels()[kernel], Config(tile_size=64, threads_per_row=8,
                                                      unroll=2, block_size=256),
                   "hip", outdir=str(tmp_path))
    so, log = compile_generated(gen, "hip", str(tmp_path))
    declared = [s for s in _declared("tilegen_launch.h")
                if not s.startswith("launch_") or s == "launch_%s" % kernel]
    exported = _exported(so)
    assert not [s for s in declared if s not in exported]
    assert "tgv_launch_async" in exported  # declared as one typedef per kernel
    runtime.lib()
    lib = ctypes.CDLL(so)
    lib.tgv_kernel_name.restype = ctypes.c_char_p
    assert lib.tgv_kernel_name().decode() == kernel
    g, b, l = ctypes.c_int64(), ctypes.c_int32(), ctypes.c_int32()
    lib.tgv_geometry.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_void_p] * 3
    assert lib.tgv_geometry(1000, 1000, 64, 5000, ctypes.byref(g), ctypes.byref(b),
                            ctypes.byref(l)) == 0
    assert b.value == 256 and g.value * gen.geometry.rows_per_block >= 1000


def test_variant_unload_releases_its_cached_module(tmp_path):
    """Unloading a variant library runs its destructor, which drops the
    runtime's module-cache entry for the library's embedded code object (so a
    later library mapped at the same address is not served the old kernel),
    and a process that exits with variants still loaded exits cleanly."""
    import _ctypes
    gen = generate(standard_kernels()["spmv"], Config(), "hip", outdir=str(tmp_path))
    so, _ = compile_generated(gen, "hip", str(tmp_path))
    L = runtime.lib()
    assert L.tg_code_release(None, 0) == 0  # nothing cached: no-op
    lib = ctypes.CDLL(so)
    _ctypes.dlclose(lib._handle)
    code = ("import ctypes, sys; sys.path.insert(0, %r); from tilegen_amd import runtime; "
            "runtime.lib(); ctypes.CDLL(%r); print('ok')" % (ROOT, so))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stderr


def test_header_signatures_match_generated_launchers():
    """Each launch_* declaration in the header is the generated launcher's
    signature, token for token."""
    text = open(os.path.join(ROOT, "include", "tilegen_launch.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {m.group(1): " ".join(m.group(0).split())
             for m in re.finditer(r"void (launch_[a-z_]+)\([^)]*\)", text)}
    assert sorted(decls) == sorted("launch_%s" % k for k in standard_kernels())
    for name in standard_kernels():
        gen = generate(standard_kernels()[name], Config(), "hip", write=False)
        assert " ".join(gen.abi_signature.split()) == decls["launch_%s" % name], name


def test_header_async_typedefs_match_generated_launchers():
    """Each tgv_launch_async_<name>_fn typedef in the header is the parameter
    list of the generated tgv_launch_async of that kernel (the stream, then the
    launch_<name> arguments), token for token, and every variant library
    exports tgv_launch_async."""
    text = open(os.path.join(ROOT, "include", "tilegen_launch.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {m.group(1): " ".join(m.group(2).split())
             for m in re.finditer(r"typedef int \(\*tgv_launch_async_([a-z_]+)_fn\)\(([^)]*)\)",
                                  text)}
    assert sorted(decls) == sorted(standard_kernels())
    for name in standard_kernels():
        gen = generate(standard_kernels()[name], Config(), "hip", write=False)
        m = re.search(r"int tgv_launch_async\(([^)]*)\)", gen.host_source)
        assert m, name
        assert " ".join(m.group(1).split()) == decls[name], name
        params = ", ".join("%s %s" % a for a in gen.abi_args)
        assert decls[name] == " ".join(("void* stream, " + params).split()), name


def test_launchers_pass_no_dynamic_lds(tmp_path):
    """Every generated kernel declares its LDS statically, so the launch asks for
    no dynamic LDS on top of it (passing the static size again would reserve it
    twice per workgroup and halve the workgroups a CU can hold)."""
    from tilegen_amd.matrices import baseline_case
    from tilegen_amd.schedules import NOALLOC_SCHEDULE, TUNED
    todo = [(baseline_case(c).kernel, cfg) for c, cfg in TUNED.items()]
    todo += [("spmv", NOALLOC_SCHEDULE),
             ("spmv", Config(tile_size=64, threads_per_row=4, unroll=2, block_size=256,
                             balance="nnz"))]
    runtime.lib()
    for kernel, cfg in todo:
        gen = generate(standard_kernels()[kernel], cfg, "hip", outdir=str(tmp_path))
        so, _ = compile_generated(gen, "hip", str(tmp_path))
        assert "__shared__" in gen.source or gen.geometry.lds_bytes == 0, cfg.short()
        assert "extern __shared__" not in gen.source
        lib = ctypes.CDLL(so)
        g, b, l = ctypes.c_int64(), ctypes.c_int32(), ctypes.c_int32(-1)
        lib.tgv_geometry.argtypes = [ctypes.c_int64] * 4 + [ctypes.c_void_p] * 3
        assert lib.tgv_geometry(100000, 100000, 64, 1600000, ctypes.byref(g), ctypes.byref(b),
                                ctypes.byref(l)) == 0
        assert l.value == 0, (cfg.short(), l.value)


def test_runtime_error_reporting_without_device():
    L = runtime.lib()
    L.tg_clear_error()
    assert L.tg_last_status() == 0 and runtime.last_error() == ""
    with pytest.raises(runtime.TileGenHipError):
        runtime.check(L.tg_launch(None, 1, 64, 0, None, 0, None, 1), "launch")
    assert "null function" in runtime.last_error()


@pytest.mark.parametrize("grid,block", [(1 << 22, 1024), ((1 << 32) // 64, 64), (1, 1025),
                                        (-1, 64), (1, 0)])
def test_launch_geometry_refused_before_any_device_call(grid, block):
    """A dispatch's grid is a 32-bit count of work-items, and a workgroup holds
    at most 1024 lanes: both launch entry points refuse anything else with an
    error before any HIP call (the function handle here is never called)."""
    L = runtime.lib()
    fake = ctypes.c_void_p(0x1000)
    key = ctypes.c_char_p(b"key")
    for name, call in (
            ("tg_launch", lambda: L.tg_launch(fake, grid, block, 0, None, 0, None, 1)),
            ("tg_launch_ordered",
             lambda: L.tg_launch_ordered(key, fake, grid, block, 0, None, 0, None, 1))):
        L.tg_clear_error()
        assert call() == -1, name
        assert "invalid geometry" in runtime.last_error(), (name, runtime.last_error())


def test_graph_entry_points_refuse_null_arguments():
    """Refused before any HIP call: the null stream cannot be captured, and a
    null graph is neither launched nor an error to destroy."""
    L = runtime.lib()
    for call, text in ((lambda: L.tg_graph_begin(None), "null stream cannot be captured"),
                       (lambda: L.tg_graph_end(None, None), "null stream"),
                       (lambda: L.tg_graph_launch(None, None, 1), "null graph")):
        L.tg_clear_error()
        assert call() == -1
        assert text in runtime.last_error()
    assert L.tg_graph_destroy(None) == 0


def test_rtc_compile_and_errors():
    code, _ = runtime.rtc_compile('extern "C" __global__ void k(double* a) { a[0] = 1.0; }',
                                  "k.hip", ["--offload-arch=gfx950", "-O3"])
    assert code[:4] == b"\x7fELF"
    with pytest.raises(runtime.TileGenHipError) as err:
        runtime.rtc_compile("this is not HIP", "bad.hip", ["--offload-arch=gfx950"])
    assert "bad.hip" in str(err.value)


def test_no_packed_fp32_in_generated_code(tmp_path):
    """Generated kernels are compiled without packed-FP32 operations."""
    objdump = "/opt/rocm/llvm/bin/llvm-objdump"
    if not os.path.exists(objdump):
        pytest.skip("llvm-objdump not available")
    for kernel in ("spmv", "spmm", "sddmm"):
        gen = generate(standard_kernels()[kernel], Config(tile_size=64, threads_per_row=8,
                                                          unroll=2, vector_width=2,
                                                          block_size=256),
                       "hip", outdir=str(tmp_path))
        so, _ = compile_generated(gen, "hip", str(tmp_path))
        co = so[:-3] + ".co"
        asm = subprocess.run([objdump, "-d", "--mcpu=gfx950", co], capture_output=True,
                             text=True).stdout
        assert "v_pk_fma_f32" not in asm and "v_pk_add_f32" not in asm and \
            "v_pk_mul_f32" not in asm
        assert "scratch_" not in asm  # no register spills


def test_tuned_schedules_do_not_spill(tmp_path):
    """The schedule every BASELINE config is benchmarked with, and the no-alloc
    schedule, keep all their values in registers: the code object's metadata
    gives no private segment and no VGPR or SGPR spills."""
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    if not os.path.exists(readelf):
        pytest.skip("llvm-readelf not available")
    from tilegen_amd.matrices import baseline_case
    from tilegen_amd.schedules import NOALLOC_SCHEDULE, TUNED
    todo = [(baseline_case(c).kernel, c, cfg) for c, cfg in TUNED.items()]
    todo.append(("spmv", "noalloc", NOALLOC_SCHEDULE))
    for kernel, label, cfg in todo:
        gen = generate(standard_kernels()[kernel], cfg, "hip", outdir=str(tmp_path))
        so, _ = compile_generated(gen, "hip", str(tmp_path))
        notes = subprocess.run([readelf, "--notes", so[:-3] + ".co"], capture_output=True,
                               text=True).stdout
        meta = dict(re.findall(r"\.(private_segment_fixed_size|vgpr_spill_count|"
                               r"sgpr_spill_count):\s+(\d+)", notes))
        assert len(meta) == 3, (label, notes[:400])
        assert all(v == "0" for v in meta.values()), (label, cfg.short(), meta)


def test_noalloc_library_code_object_does_not_spill(tmp_path):
    """libtgna's own kernels, compiled by hipcc with the library's flags (not the
    hipRTC build of the same schedule above), keep every value in registers."""
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    if not os.path.exists(readelf):
        pytest.skip("llvm-readelf not available")
    from tilegen_amd.build import noalloc_code_object
    co = noalloc_code_object(str(tmp_path / "libtgna_device.co"))
    notes = subprocess.run([readelf, "--notes", co], capture_output=True, text=True).stdout
    kernels = re.split(r"\n\s+- \.", notes)
    found = {}
    for k in kernels:
        name = re.search(r"\.name:\s+(\S+)", k)
        if not name:
            continue
        meta = dict(re.findall(r"\.(private_segment_fixed_size|vgpr_spill_count|"
                               r"sgpr_spill_count):\s+(\d+)", k))
        found[name.group(1)] = meta
    assert "spmv_kernel" in found and any("tg_na_clear" in n for n in found), sorted(found)
    for name, meta in found.items():
        assert len(meta) == 3 and all(v == "0" for v in meta.values()), (name, meta)


def test_noalloc_library_exports_its_header():
    """libtgna.so exports exactly what include/tilegen_noalloc.h declares and
    loads without a GPU."""
    import os as _os
    path = _os.path.join(runtime.lib_dir(), "libtgna.so")
    declared = _declared("tilegen_noalloc.h")
    assert declared == ["launch_spmv_noalloc"]
    exported = _exported(path)
    assert sorted(exported & set(declared)) == declared
    assert not [s for s in exported if s.startswith(("tg_", "tgv_", "spmv_"))]
    L = runtime.noalloc_lib()
    assert L.launch_spmv_noalloc.restype is ctypes.c_int
