// Kernel choice of the grouped GEMM entry points (capi.hip): the checked
// parameters of a descriptor, the route (kernel path, token tile, K split,
// workspace) and the launch along it.
#pragma once

#include "../../include/qmoe.h"
#include "gemm_common.h"

struct QmoeRoute {
  int path = 0;    // 0 streaming, 1 1-byte tiles, 2 4-bit tiles, 3 generic tiles, 4 streaming passes,
                   // 5 1-byte tiles on persistent workgroups, 6 MX (e2m1 x e2m1) persistent tiles,
                   // 7 MX grouped tiles, 8 streaming with the activation quantization inside,
                   // 9 1-byte tiles of 128 weight rows, 10 streaming in row slices (one per grid.z)
  int tile_m = 0;  // token rows per tile (tiled) or per pass (streaming)
  int ksplit = 1;
  int64_t ws_bytes = 0;  // split-K partials the launch needs
};

// Descriptor -> kernel parameters; QMOE_ERR_ARG for a bad descriptor.
int qmoe_to_params(const qmoe_gemm_desc* d, GemmParams* p);
// The kernel qmoe_gemm runs for the problem (clears the active list in `p`
// for the tiled kernels); QMOE_ERR_ARG when no kernel takes it.
int qmoe_route_of(const qmoe_gemm_desc* d, GemmParams& p, QmoeRoute* r);
// Launch along the route with `workspace` (>= r.ws_bytes when r.ksplit > 1).
int qmoe_run_route(const qmoe_gemm_desc* d, const QmoeRoute& r, GemmParams p, void* workspace,
                   int64_t ws_bytes, hipStream_t stream);
