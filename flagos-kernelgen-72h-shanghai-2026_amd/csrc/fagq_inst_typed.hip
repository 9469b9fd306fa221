// fagq_inst_typed.hip - the typed form's kernels for one (code format, scale
// format) pair, selected with -DFAGQ_QF=<0|1|2> -DFAGQ_SF=<0|1>: fagq_rows
// with fp16 elements (every group size, steps per wave, norm_out choice and
// row-group mode, as fagq_inst.hip has for bf16) and fagq_rows_typed for the
// families with an fp32 tensor, and their launch lookups.
#include "fagq_dispatch.hpp"

#ifndef FAGQ_QF
#error "FAGQ_QF must be defined"
#endif
#ifndef FAGQ_SF
#error "FAGQ_SF must be defined"
#endif

#define FAGQ_CAT4(a, b, c, d) a##b##c##d
#define FAGQ_LOOKUP_TYPED(q, s) FAGQ_CAT4(lookup_typed_q, q, _s, s)
#define FAGQ_LOOKUP_F16(q, s) FAGQ_CAT4(lookup_f16_q, q, _s, s)

namespace fagq {
namespace {

template <int NS, int LPG, bool NORM, int MODE>
int launch_rows_f16(const KArgs& a, dim3 grid, dim3 block, unsigned lds, hipStream_t stream) {
  void* args[] = {const_cast<KArgs*>(&a)};
  return launch_kernel(
      reinterpret_cast<const void*>(&fagq_rows<NS, LPG, FAGQ_QF, FAGQ_SF, NORM, MODE, ET_F16>),
      grid, block, args, lds, stream);
}

template <int NS, int LPG, bool NORM, int TF>
int launch_typed(const KArgs& a, dim3 grid, dim3 block, unsigned lds, hipStream_t stream) {
  void* args[] = {const_cast<KArgs*>(&a)};
  return launch_kernel(
      reinterpret_cast<const void*>(&fagq_rows_typed<NS, LPG, FAGQ_QF, FAGQ_SF, NORM, TF>), grid,
      block, args, lds, stream);
}

}  // namespace

#define FAGQ_R16(NS, LPG, NORM) \
  {&launch_rows_f16<NS, LPG, NORM, RG_INDEPENDENT>, &launch_rows_f16<NS, LPG, NORM, RG_SHARED_GAMMA>, \
   &launch_rows_f16<NS, LPG, NORM, RG_WIDE_SCALES>}
#define FAGQ_N16(NS, LPG) {FAGQ_R16(NS, LPG, false), FAGQ_R16(NS, LPG, true)}
#define FAGQ_S16(LPG) {FAGQ_N16(1, LPG), FAGQ_N16(2, LPG), FAGQ_N16(3, LPG), FAGQ_N16(4, LPG)}

static_assert(kMaxStepsPerWave == 4, "FAGQ_S16 lists 4 step counts");
static_assert(kNumModes == 3, "FAGQ_R16 lists 3 row-group modes");

LaunchFn FAGQ_LOOKUP_F16(FAGQ_QF, FAGQ_SF)(int lpg_idx, int steps, bool norm, int mode) {
  static const LaunchFn table[kNumLpg][kMaxStepsPerWave][2][kNumModes] = {
      FAGQ_S16(8), FAGQ_S16(16), FAGQ_S16(32)};
  return table[lpg_idx][steps - 1][norm ? 1 : 0][mode];
}

// Families with an fp32 tensor, in TypeFamily order from TF_BF16_R32.
#define FAGQ_T(NS, LPG, NORM) \
  {&launch_typed<NS, LPG, NORM, TF_BF16_R32>, &launch_typed<NS, LPG, NORM, TF_F16_R32>, \
   &launch_typed<NS, LPG, NORM, TF_F32>}
#define FAGQ_TN(NS, LPG) {FAGQ_T(NS, LPG, false), FAGQ_T(NS, LPG, true)}
#define FAGQ_TS(LPG) {FAGQ_TN(1, LPG), FAGQ_TN(2, LPG), FAGQ_TN(3, LPG), FAGQ_TN(4, LPG)}

static_assert(kNumTypeFamilies == 4 && TF_BF16_R32 == 1 && TF_F32 == 3,
              "FAGQ_T lists the families TF_BF16_R32 .. TF_F32");

LaunchFn FAGQ_LOOKUP_TYPED(FAGQ_QF, FAGQ_SF)(int lpg_idx, int steps, bool norm, int family) {
  static const LaunchFn table[kNumLpg][kMaxStepsPerWave][2][kNumTypeFamilies - 1] = {
      FAGQ_TS(8), FAGQ_TS(16), FAGQ_TS(32)};
  return table[lpg_idx][steps - 1][norm ? 1 : 0][family - TF_BF16_R32];
}

}  // namespace fagq
