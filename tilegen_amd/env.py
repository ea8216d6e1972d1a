"""Toolchain and GPU probe that picks the backend (reference ``tilegen/env.py``).

``probe()`` never raises.  The HIP backend needs a gfx950-capable hipRTC
(libtgrt built in-tree) *and* a visible AMD GPU; otherwise the backend is
"cpu".  GPU detection reads the KFD topology in sysfs, so probing does not
initialise the HIP runtime; ``probe(deep=True)`` also asks HIP for the device
name and CU count.  The reference's CUDA keys (``has_nvcc``, ``sm_arch`` ...)
are kept, always empty, so callers that read them still work.
"""

from __future__ import annotations

import glob
import json
import os
import platform
import shutil
import subprocess
from typing import Dict, List, Optional

__all__ = ["probe", "cpu_name", "num_cores", "physical_cores", "pretty", "kfd_gpus"]


def _run(cmd: List[str], timeout: float = 10.0) -> Optional[str]:
    try:
        out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                             timeout=timeout, check=False)
        if out.returncode != 0:
            return None
        return out.stdout.decode("utf-8", "replace").strip()
    except Exception:
        return None


def cpu_name() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine() or "unknown"


def num_cores() -> int:
    try:
        return int(os.cpu_count() or 1)
    except Exception:
        return 1


def physical_cores() -> int:
    """Distinct (physical id, core id) pairs in /proc/cpuinfo."""
    try:
        pairs, phys, core = set(), None, None
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                key, _, val = line.partition(":")
                key = key.strip()
                if key == "physical id":
                    phys = val.strip()
                elif key == "core id":
                    core = val.strip()
                elif not key and phys is not None:
                    pairs.add((phys, core))
                    phys = core = None
        if phys is not None:
            pairs.add((phys, core))
        return len(pairs) or num_cores()
    except Exception:
        return num_cores()


def kfd_gpus() -> List[Dict[str, object]]:
    """GPU nodes of the KFD topology (``simd_count > 0``) with their gfx target."""
    gpus = []
    for props in sorted(glob.glob("/sys/class/kfd/kfd/topology/nodes/*/properties")):
        try:
            kv = {}
            with open(props) as fh:
                for line in fh:
                    parts = line.split()
                    if len(parts) == 2:
                        kv[parts[0]] = parts[1]
            if int(kv.get("simd_count", "0")) <= 0:
                continue
            ver = int(kv.get("gfx_target_version", "0"))
            major, minor, step = ver // 10000, (ver // 100) % 100, ver % 100
            gpus.append({"gfx": "gfx%d%d%x" % (major, minor, step) if ver else None,
                         "simd_count": int(kv.get("simd_count", "0")),
                         "node": os.path.basename(os.path.dirname(props))})
        except Exception:
            continue
    return gpus


def _hip_version() -> Optional[str]:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        return None
    text = _run([exe, "--version"])
    if not text:
        return None
    for line in text.splitlines():
        if line.startswith("HIP version"):
            return line.split(":", 1)[1].strip()
    return text.splitlines()[0]


def probe(deep: bool = False) -> Dict[str, object]:
    """Keys: has_hiprtc, hip_version, has_gpu, gpu_name, gfx_arch, cu_count,
    cpu_name, num_cores, physical_cores, backend, plus the reference's CUDA
    keys (always empty here)."""
    info: Dict[str, object] = {
        "has_hiprtc": False, "hip_version": None, "has_gpu": False, "gpu_name": None,
        "gfx_arch": None, "cu_count": None, "cpu_name": "unknown", "num_cores": 1,
        "physical_cores": 1, "backend": "cpu",
        "has_nvcc": False, "nvcc_version": None, "compute_capability": None, "sm_arch": None,
    }
    try:
        from . import runtime
        info["has_hiprtc"] = os.path.exists(runtime.lib_path()) and bool(
            glob.glob("/opt/rocm*/lib/libhiprtc.so*"))
    except Exception:
        pass
    try:
        info["hip_version"] = _hip_version()
    except Exception:
        pass
    try:
        gpus = kfd_gpus()
        if gpus:
            info["has_gpu"] = True
            info["gfx_arch"] = gpus[0]["gfx"]
    except Exception:
        pass
    if deep and info["has_gpu"] and info["has_hiprtc"]:
        try:
            from . import runtime
            d = runtime.device_info(0)
            info["gpu_name"] = d["name"] or d["arch"]
            info["gfx_arch"] = d["arch"].split(":")[0]
            info["cu_count"] = d["cu_count"]
        except Exception:
            pass
    info["cpu_name"] = cpu_name()
    info["num_cores"] = num_cores()
    info["physical_cores"] = physical_cores()
    if info["has_gpu"] and info["has_hiprtc"]:
        info["backend"] = "hip"
    return info


def pretty(info: Optional[Dict[str, object]] = None) -> str:
    info = probe() if info is None else info
    keys = ["backend", "cpu_name", "num_cores", "physical_cores", "has_hiprtc", "hip_version",
            "has_gpu", "gpu_name", "gfx_arch", "cu_count"]
    return "\n".join(["TileGen environment probe", "-------------------------"] +
                     ["%-14s: %s" % (k, info.get(k)) for k in keys])


if __name__ == "__main__":  # pragma: no cover
    print(json.dumps(probe(deep=True), indent=2))
