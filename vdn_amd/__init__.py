"""vdn_amd: MI355X-native (gfx950) hot path of the VDN-H3 hybrid-attention DiT block.

Host code mirrors the reference's operator API (MXFP8 producers and linears, VDA
linear-attention ops, frame-window softmax attention, QK RMSNorm + 3D RoPE) and calls
hand-written HIP kernels in libvdnmi.so through a C ABI (include/vdnmi.h).
"""
__all__ = ["mxfp8"]
