// g2b_tiles.hip - launchers of k_tiles (g2b_tiles.h), the decode kernel whose
// K scores run on the int8 matrix cores (Q8_0 KV, head_dim 128, 8 KV heads,
// 3 or 4 q heads per KV head).
#include "g2b_tiles.h"

namespace g2b {

bool tiles_available(const ShapeDev &sh) {
  return tiles_shape_ok(sh) && sh.n_heads * sh.head_dim <= 8192;
}

template <int G, bool WQ>
static hipError_t launch_tiles_g(const DecodeParams &p, int n_layers, hipStream_t s) {
  const dim3 grid = WQ ? dim3(p.wq_grid) : static_grid(p, n_layers);
  hipLaunchKernelGGL((k_tiles<G, WQ>), grid, dim3(kThreads), tiles_lds_layout(p.sh).total, s, p);
  return hipGetLastError();
}

hipError_t launch_tiles(const DecodeParams &p, int n_layers, hipStream_t s) {
  if (!tiles_available(p.sh) || p.att) return hipErrorInvalidValue;
  const int g = p.sh.n_heads / p.sh.n_kv_heads;
  if (g == 4) return p.wq ? launch_tiles_g<4, true>(p, n_layers, s) : launch_tiles_g<4, false>(p, n_layers, s);
  return p.wq ? launch_tiles_g<3, true>(p, n_layers, s) : launch_tiles_g<3, false>(p, n_layers, s);
}

template <int G, bool WQ>
static int tiles_occ(const ShapeDev &sh) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_tiles<G, WQ>, kThreads,
                                                   tiles_lds_layout(sh).total) != hipSuccess) {
    (void)hipGetLastError();
    return 1;
  }
  return n > 0 ? n : 1;
}

int tiles_blocks_per_cu(const ShapeDev &sh, bool wq) {
  if (!tiles_available(sh)) return 1;
  const int g = sh.n_heads / sh.n_kv_heads;
  if (g == 4) return wq ? tiles_occ<4, true>(sh) : tiles_occ<4, false>(sh);
  return wq ? tiles_occ<3, true>(sh) : tiles_occ<3, false>(sh);
}

}  // namespace g2b
