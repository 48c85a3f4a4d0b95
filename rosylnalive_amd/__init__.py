"""rosylnalive_amd: an MI355X-native (gfx950) backend for the Qwen3 decoder forward of enderPeer/rosylnalive.

The product is the C-ABI library liblrm_hip.so (HIP kernels + a HIP device behind the reference's Lrm.Gpu.Core
contract + a Qwen3 executor). The Python modules here are thin ctypes front ends over that library.
"""
