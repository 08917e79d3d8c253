// Single translation unit for the gfx950 code object (hayai_kernels.hsaco).
#include "gemv.hip"
#include "q4k.hip"
#include "lut.hip"
#include "q4k_ffn.hip"
#include "q4k_mm.hip"
#include "moe.hip"
#include "dequant.hip"
#include "synth.hip"
