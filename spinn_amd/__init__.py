"""spinn_amd - SPINN's convolution / GEMM hot path on MI355X (gfx950).

The product is the native library ``spinn_amd/lib/libspinn.so``: hand-written
HIP kernels behind the C ABI of include/spinn_hip.h, and the C host runtime of
include/spinn_runtime.h (ENNF load -> plan -> run over one HBM arena). This
package adds the build script, ctypes bindings and the seeded ENNF model
generators used by the tests and the benchmark.
"""
from . import ennf, models  # noqa: F401

__all__ = ["ennf", "models", "native", "build"]
