"""fable5_llm_amd -- MI355X-native W4A8 matvec engine.

A drop-in for the matvec datapath of coreyhahn/fable5_llm: the integer law
of ref/w4a8_ref.py / ref/fixedpoint.py / ref/layer_fixed.py executed by
hand-written HIP kernels for gfx950 behind the C ABI of
include/fable5_w4a8.h.

  engine        Context / Weights handle API (host and device buffers)
  w4a8_ref      matvec_y32, rshift_round, row image packing (reference names)
  fixedpoint    dyn_quant_i8
  layer_fixed   matvec_fx, matvec_to, rmsnorm_fx, mlp_fx, MOVY/ALU ops, head
  stream9b      the Qwen3.5-9B-shaped decode weight stream (249 matrices)
  build         hipcc build of libfable5_w4a8.so
"""
__all__ = ["engine", "w4a8_ref", "fixedpoint", "layer_fixed", "stream9b"]
