"""santa_amd -- MI355X-native S^2ANTA sampled-attention decode.

Layout:
  santa_amd/csrc/            HIP kernels (gfx950), the C ABI, the torch extension sources
  santa_amd/libsanta_amd.so  the built library (include/santa_amd.h)
  santa_amd/attention_backends.py  the reference's decode-backend adapter contract
  santa_flash_batch_cuda, santa_prop_batch_cuda  drop-in extension packages (repo root)
"""
__version__ = "0.1.0"
