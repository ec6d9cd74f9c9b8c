"""llmplayer_amd -- MI355X-native decode/prefill attention path for LLMPlayer.

The compute lives in libllmp_hip.so (HIP, gfx950), declared by include/llmp_hip.h.  This
package holds its build recipe (csrc/Makefile), the ctypes binding (_lib) and the host-side
mirror of the reference's GPU attention section (hip_forward_pass.HipForwardPass).
"""
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))


def build() -> str:
    """Compile libllmp_hip.so for gfx950 (always recompiles)."""
    subprocess.run(["make", "-B", "-C", os.path.join(_HERE, "csrc")], check=True)
    return os.path.join(_HERE, "libllmp_hip.so")
