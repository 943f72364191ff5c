// decode_mega.h -- arguments of the one-kernel decode layer (decode_mega.hip) and its
// host entry points, shared with the layer orchestration in decode.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nve_kernels.h"

namespace nve {
namespace mega {

struct Args {
  int H, QD, KD, F, D, heads, kv_heads, max_seq, xcd_map, red_off;
  float eps, qscale;
  const uint8_t* nib[7];  // q k v o gate up down
  const float* sc[7];
  const uint16_t* norm1;
  const uint16_t* norm2;
  float* h;
  uint16_t* kc;
  uint16_t* vc;
  const int* pos;
  const float* rcos;
  const float* rsin;
  float* q;
  float* k;
  float* v;
  float* part;
  float* hmid;
  float* mid;
  unsigned* bar;
  unsigned long long* trace;  // NULL, or [grid][16] phase timestamps (diagnostics)
};

}  // namespace mega
}  // namespace nve

namespace nve_host {
// Bytes of the grid-barrier words in the decode workspace.
size_t mega_bar_bytes();
// Compiled shape class for this layer configuration and key split, or -1.
int mega_class(const nve_decode_config& c, int split);
hipError_t launch_layer_mega(int cls, bool w4a8, int split, const nve::mega::Args& a, hipStream_t s);
}  // namespace nve_host
