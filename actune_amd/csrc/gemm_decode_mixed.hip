// The decode kernel over sibling linears of different weight widths (one
// activation width): q/k/v or gate/up of a mixed-precision bank in one
// launch instead of one launch per width. A workgroup's problem (blockIdx.y)
// names its width, and the workgroup runs that width's body of the decode
// kernel (decode_body.hpp): the activation slab is private to the workgroup,
// so each workgroup lays the quantized activations out in its own width's
// operand order, and every output equals the single-width launch bit for
// bit. The bodies run without the full-ring specialisation (bounds-tested
// slot loop), and the row tiles per workgroup are the fewest any width needs.
#include "decode_body.hpp"

namespace actune {

template <int A, int NW, int MT, bool PACKED, bool SCALE, bool ONE, int TR>
__global__ __launch_bounds__(NW * 64) void gemm_decode_mixed(const LinearArgs args, int GW) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int w = args.prob[blockIdx.y].W;  // uniform over the workgroup
  if (w == 8) decode_tile<8, A, NW, decode_ring(8) / TR, MT, PACKED, SCALE, ONE, false, TR>(args, GW, smem);
  else if (w == 4) decode_tile<4, A, NW, decode_ring(4) / TR, MT, PACKED, SCALE, ONE, false, TR>(args, GW, smem);
  else decode_tile<2, A, NW, decode_ring(2) / TR, MT, PACKED, SCALE, ONE, false, TR>(args, GW, smem);
}

namespace {

template <int A, int NW, int MT, bool PACKED, bool SCALE, bool ONE, int TR>
void launch_mixed_one(const LinearArgs& g, hipStream_t st) {
  const size_t lds = decode_lds_bytes(g.K, g.M, NW, TR);
  allow_dynamic_lds<gemm_decode_mixed<A, NW, MT, PACKED, SCALE, ONE, TR>>();
  const int groups = (decode_max_tiles(g) + TR - 1) / TR, blocks = MT == 16 ? (g.M + 15) / 16 : 1;
  gemm_decode_mixed<A, NW, MT, PACKED, SCALE, ONE, TR>
      <<<dim3((unsigned)groups, (unsigned)g.nprob, (unsigned)blocks), NW * 64, lds, st>>>(
          g, decode_groups_per_wave(g.K, NW));
}

// M > 1: the row tiles per workgroup that every width's ring holds
template <int A, int NW, int MT, bool PACKED, bool SCALE>
void launch_mixed_tr(const LinearArgs& g, hipStream_t st) {
  const int blocks = MT == 16 ? (g.M + 15) / 16 : 1;
  int tr = 4;
  for (int q = 0; q < g.nprob; ++q)
    tr = std::min(tr, decode_row_tiles(g.K, g.M, g.prob[q].W, NW, decode_max_tiles(g), g.nprob * blocks, false));
  if (tr == 4) launch_mixed_one<A, NW, MT, PACKED, SCALE, false, 4>(g, st);
  else if (tr == 2) launch_mixed_one<A, NW, MT, PACKED, SCALE, false, 2>(g, st);
  else launch_mixed_one<A, NW, MT, PACKED, SCALE, false, 1>(g, st);
}

template <int A, int NW, bool PACKED, bool SCALE>
void launch_mixed_m(const LinearArgs& g, hipStream_t st) {
  if (g.M == 1) launch_mixed_one<A, NW, 4, PACKED, SCALE, true, 1>(g, st);
  else if (g.M <= 4) launch_mixed_tr<A, NW, 4, PACKED, SCALE>(g, st);
  else if (g.M <= 8) launch_mixed_tr<A, NW, 8, PACKED, SCALE>(g, st);
  else launch_mixed_tr<A, NW, 16, PACKED, SCALE>(g, st);
}

template <int A, int NW>
void launch_mixed_nw(bool packed, const LinearArgs& g, hipStream_t st) {
  if (packed) launch_mixed_m<A, NW, true, false>(g, st);
  else if (g.xscale) launch_mixed_m<A, NW, false, true>(g, st);
  else launch_mixed_m<A, NW, false, false>(g, st);
}

template <int A>
void launch_mixed_a(int nw, bool packed, const LinearArgs& g, hipStream_t st) {
  if (nw == 4) launch_mixed_nw<A, 4>(packed, g, st);
  else if (nw == 8) launch_mixed_nw<A, 8>(packed, g, st);
  else launch_mixed_nw<A, 16>(packed, g, st);
}

}  // namespace

void launch_decode_mixed(int A, int nw, bool packed, const LinearArgs& g, hipStream_t st) {
  if (A == 8) launch_mixed_a<8>(nw, packed, g, st);
  else if (A == 4) launch_mixed_a<4>(nw, packed, g, st);
  else launch_mixed_a<2>(nw, packed, g, st);
}

}  // namespace actune
