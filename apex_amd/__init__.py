"""APEX NVFP4 matmul path on MI355X (gfx950): HIP kernels behind a C ABI
(include/apex_hip.h, apex_amd/csrc), the C++ host layer (apex_amd/host) and the
Python plumbing used by tests and the benchmark (apex_amd.hip, apex_amd.synth)."""
