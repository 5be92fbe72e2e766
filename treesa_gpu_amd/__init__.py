"""MI355X-native TreeSA sweep path: HIP kernels for gfx950 behind a C ABI (include/treesa_hip.h), a C++ host
binary that is a drop-in for the reference's treesa_gpu CLI (bin/treesa_gpu), and ctypes bindings of both
(capi, host) for tests and benchmarks."""
import os

HERE = os.path.dirname(os.path.abspath(__file__))
BINARY = os.path.join(HERE, "bin", "treesa_gpu")
