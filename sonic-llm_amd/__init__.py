"""sonic-llm_amd: an MI355X-native batched decode/verify step behind the sllm-next C ABI (include/sn.h).

The product is libsn_hip.so (csrc/: HIP kernels for gfx950 and the C ABI). sllm_next.py is its Python binding. The
directory name is not a Python identifier; code that wants the binding puts this directory on sys.path and imports
`sllm_next`.
"""
