"""mica_amd -- the W8A8 linear-layer hot path of akivet/Mica's prefill-only scoring runtime,
rebuilt for AMD Instinct MI355X (gfx950) as hand-written HIP kernels behind a C ABI
(include/mica_amd.h, libmica_amd.so) with the reference's Python operator surface on top:

  int8_kernels   act_quant / mm_i8 / available / preload / STATS   (lib/int8_kernels.py)
  fused_kernels  rms_norm / swi_glu / rms_norm_quant               (lib/fused_kernels.py)
  int8_runtime   QLinear, GateUpQLinear, W8A8MLP, selftest         (lib/int8_runtime.py)
  readout        LabelReadout                                     (lib/release_runtime.py:298-306)
  model          synthetic 4B-shaped W8A8 stack (prefill + last-position readout)
"""
__version__ = "0.1.0"
