// kernels.hip — the one translation unit of the gfx950 code object
// (kernels.hsaco), loaded at run time with hipModuleLoad.
#include "gemv.hip"
#include "prim.hip"
#include "attn.hip"
#include "gemm.hip"
#include "rows.hip"
