"""GLoRCQ's quantized-linear hot path on MI355X (gfx950): HIP kernels behind a
C ABI (include/glorcq_hip.h, glorcq_amd/lib/libglorcq_hip.so), torch.library
operators over them (glorcq_amd.ops, namespace glorcq_hip), and host modules
that mirror the reference's inference package (kernels, quantized_linear,
moe_block, graph_wrapper, model_builder, hadamard_rotation)."""

from . import ops  # noqa: F401  (registers the glorcq_hip operators)
