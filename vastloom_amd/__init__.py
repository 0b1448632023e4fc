"""MI355X-native quantized routed-expert path (HIP kernels behind a C ABI).

The compute lives in ``libvastloom_hip.so`` (built by ``python -m vastloom_amd.build``); the
Python modules here are thin views over its C ABI: ``ops`` (device matrices, matvec, expert FFN,
MoE layer), ``workloads`` (seeded synthetic inputs).
"""

__all__ = ["ops", "workloads"]
