"""MI355X-native (gfx950) decode-time retrieval path of LAPrune.

Layout:
  csrc/        hand-written HIP kernels + the C ABI (include/laprune_hip.h)
  _native.py   ctypes binding of the C ABI (fails loudly when not built)
  aq_kernels/  drop-in for the reference's ``aq_kernels`` package
  attention.py drop-in ``do_sdpa_attn``
  aq_kv.py     codebook manager (scoring / encode dispatch, codebook loader)
  retrieval.py decode-step retrieval: selection arithmetic, keep set, pipeline
"""
__version__ = "0.1.0"
