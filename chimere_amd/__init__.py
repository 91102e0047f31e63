"""chimere_amd -- MI355X (gfx950) decode-time quantized GEMV / MoE-FFN path.

The compute lives in libchimere_hip.so (HIP kernels behind the C ABI of
include/chimere_hip.h); this package is the host-side binding:

* ``chimere_amd.ggml_gpu`` -- mirror of the reference's Rust wrapper module
  (chimere-server/src/kernels/ggml_gpu.rs) over the C ABI;
* ``chimere_amd.moe`` -- ``MoeLayer``: one routed-MoE FFN layer (decode and
  prefill) with its preallocated workspace.
"""
from ._lib import IQ3_S, Q4_0, Q8_0, ChimereError, lib  # noqa: F401
