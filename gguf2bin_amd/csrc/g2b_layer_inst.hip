// g2b_layer_inst.hip - one (KV format, head_dim, GQA group) instantiation of
// k_layer's launchers.  The build compiles this file once per combination
// with -DG2B_FMT=<0|1> -DG2B_HD=<64|128> -DG2B_G=<1..4>.
#include "g2b_layer.h"

#if !defined(G2B_FMT) || !defined(G2B_HD) || !defined(G2B_G)
#error "g2b_layer_inst.hip needs -DG2B_FMT, -DG2B_HD and -DG2B_G"
#endif

namespace g2b {
template hipError_t launch_layer<G2B_FMT, G2B_HD, G2B_G>(const DecodeParams &, int, hipStream_t);
template int layer_occupancy<G2B_FMT, G2B_HD, G2B_G>(const ShapeDev &, int32_t, int32_t, int32_t,
                                                     bool);
}  // namespace g2b
