"""The benchmark's measuring stick, kept out of the product: a plain
streaming-read kernel (stream_probe.hip) built into its own library,
bench_probe/libstream_probe.so, that only bench.py loads."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "stream_probe.hip")
LIB = os.path.join(HERE, "libstream_probe.so")


def build(verbose: bool = True) -> str:
    """Compile stream_probe.hip for gfx950 into libstream_probe.so."""
    from shady_thinker_amd.build import FLAGS, HIPCC

    tmp = LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, "-shared", SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {SRC}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB
