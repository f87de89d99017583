"""gfx950 device assembly of the library's sources, for the CPU tests that
check properties of the generated code.

Each csrc/*.hip is compiled once per test process with the Makefile's
HIPFLAGS (read from the Makefile, so the listing is the code the library
ships) plus ``--cuda-device-only -S``; all sources compile in parallel on the
first request.
"""
from __future__ import annotations

import os
import re
import shlex
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fused-logprob-entropy-cuda-kernel-for-llm-post-training_amd")
CSRC = os.path.join(PKG, "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

_cache: dict[str, str] = {}


def available() -> bool:
    return bool(shutil.which(HIPCC)) or os.path.exists(HIPCC)


def sources() -> list[str]:
    return sorted(n for n in os.listdir(CSRC) if n.endswith(".hip"))


def hipflags() -> list[str]:
    """HIPFLAGS of the Makefile (continuation lines joined, $(ARCH)
    expanded)."""
    with open(os.path.join(PKG, "Makefile")) as f:
        text = f.read().replace("\\\n", " ")
    arch = re.search(r"^ARCH \?= *(\S+)", text, re.M).group(1)
    flags = re.search(r"^HIPFLAGS := *(.*)$", text, re.M).group(1)
    return shlex.split(flags.replace("$(ARCH)", arch))


def _compile(name: str, out_dir: str) -> str:
    out = os.path.join(out_dir, name + ".s")
    subprocess.run([HIPCC, *hipflags(), "--cuda-device-only", "-S",
                    os.path.join(CSRC, name), "-o", out],
                   check=True, capture_output=True, timeout=900)
    with open(out) as f:
        return f.read()


def listing(name: str) -> str:
    """Device assembly of csrc/<name> (all sources are compiled on the first
    call)."""
    if not _cache:
        names = sources()
        with tempfile.TemporaryDirectory() as d, \
                ThreadPoolExecutor(max_workers=min(8, len(names))) as pool:
            for n, text in zip(names, pool.map(lambda n: _compile(n, d), names)):
                _cache[n] = text
    return _cache[name]
