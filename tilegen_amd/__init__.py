"""TileGen for MI355X: the CSR sparse kernels (SpMV, SpMM, SDDMM) of TileGen's
DSL, pass pipeline and autotuner, lowered by a HIP emitter to gfx950 kernels
that are compiled at run time with hipRTC and launched through a C ABI.

Modules keep the reference's names and entry points:
    dsl, ir, passes   index-notation frontend, IR, schedule pipeline
    codegen           HIP (gfx950) and OpenMP emitters, ``generate``
    verify            hipRTC/g++ compilation, launch, SciPy differential check
    autotune          CDNA4 schedule search timed with GPU events
    matrices          reference corpus and the BASELINE inputs
    env               toolchain / GPU probe
    runtime           ctypes binding of libtgrt (include/tgrt.h)

Around them (the reference's scripts/ and harness, rebuilt for this backend):
    variant           one compiled variant: launch, geometry, timing handles
    schedules         tuned schedule per BASELINE case, test schedules
    verify_all        every kernel x schedule x corpus class, injected bugs
    tune_all          corpus autotune into results/
    ablation          per-pass contribution (code diff, verify, GPU timing)
    vendor            rocSPARSE SpMV timing beside the tuned kernel
    profiling         rocprofv3 summaries for profiles/
    cpu_tuned         CPU-tuned OpenMP schedules for the CPU baseline
    build             in-tree native build (libtgrt, harness, oracle, kernel cache)
"""

__version__ = "0.1.0"

__all__ = ["__version__"]
