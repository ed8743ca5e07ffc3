// The single gfx950 code object of the library: every kernel the runtime
// launches, built with
//   hipcc --offload-arch=gfx950 --offload-device-only --no-gpu-bundle-output
#include "cab.hip"
#include "attn.hip"
#include "attnx.hip"
#include "conv.hip"
#include "gemm.hip"
#include "gemmx.hip"
#include "tailx.hip"
#include "mlp.hip"
#include "habtail.hip"
#include "convw.hip"
#include "convwino.hip"
#include "misc.hip"
#include "convfirst.hip"
