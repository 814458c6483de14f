// Host side of the per-CU gate/up kernel (dspark_moe_cu.h): the plan, the launch and the plan
// query. A translation unit of its own: its unit loops are unrolled in full (up to 68 steps of
// one 1 KB load each), beyond LLVM's default threshold for a full unroll, and the build raises
// that threshold for this file only (a loop left partly rolled indexes its load window with a
// run-time index and keeps it in scratch memory).
#include <mutex>

#include "dspark_moe_cu.h"

namespace dspark {
namespace {

constexpr int kMoeCuGrid = 256;  // one workgroup per CU of MI355X; with E <= 256 experts a CU's
                                 // range of units then spans at most two experts

// The kernel reads weights and scales through buffer resources with 32-bit offsets below 2^31
bool offsets_fit(long E, long N, long K, int bits) {
  return E * N * K * bits / 8 < (1L << 31) && E * N * (K / 64) * 2 < (1L << 31);
}

// Waves per CU and loads in flight per wave (a divisor of a few units' loads, moe_cu_trip_units).
// Measured at the 30B-A3B block (K = 2048, 4 bits, 89 live experts, about 17 units per CU),
// with the per-wave seed table: 9 waves with 6 loads each, 30.9 us per launch; 6 loads per
// wave at 8 / 10 / 11 / 12 waves 34.1 / 31.3 / 31.6 / 32.2 us, and at 12 waves 4 / 9 / 12 / 18
// loads 33.1 / 33.5 / 34.6 / 36.0 us. At 8 bits (68 loads per unit) 17 loads: 50.5 us against
// 54.1 / 66.2 / 69.1 us for 8 / 6 / 12.
constexpr int kMoeCuWaves = 9;
template <int BITS, int G>
constexpr int moe_cu_window() {
  if (G == 32) return BITS == 4 ? 6 : 17;  // loads per unit: 36; 68
  return BITS == 4 ? 12 : 10;               // 12; 20
}

template <int BITS, int G, int KW>
int launch_t(const MoeCuArgs& a, hipStream_t s) {
  constexpr int PF = moe_cu_window<BITS, G>();
  static_assert(moe_cu_trip_units(moe_cu_loads<BITS, G>(), PF) > 0, "window");
  constexpr size_t lds = moe_cu_lds_bytes<G, kMoeCuWaves>();
  static_assert(lds <= 160 * 1024, "LDS of one CU");
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_cu_kernel<BITS, G, KW, PF, kMoeCuWaves>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  });
  if (attr != hipSuccess)
    return fail(DSPARK_ERR_LAUNCH, "moe_switch_glu_packed: LDS attribute: %s", hipGetErrorString(attr));
  hipLaunchKernelGGL((moe_cu_kernel<BITS, G, KW, PF, kMoeCuWaves>), dim3(kMoeCuGrid), dim3(64 * kMoeCuWaves), lds,
                     s, a);
  return check_launch("moe gate/up");
}

}  // namespace

// M <= 16 tokens, E <= 256 experts, M * k <= 512 pairs and the instantiated K = H: 2048 (two K
// parts, as rc_plan cuts it) or 512 (one)
bool moe_cu_gate_up(long M, long H, long I, long E, long k, int bits) {
  if (M > kMoeCuRows || E > kMoeCuMaxE || M * k > kMoeCuMaxPairs || (bits != 4 && bits != 8)) return false;
  return (H == 2048 || H == 512) && offsets_fit(E, I, H, bits);
}

int launch_moe_cu(const MoeCuArgs& a, long K, int bits, hipStream_t s) {
  const bool b4 = bits == 4;
  if (K == 2048) return b4 ? launch_t<4, 32, 2>(a, s) : launch_t<8, 32, 2>(a, s);
  if (K == 512) return b4 ? launch_t<4, 8, 1>(a, s) : launch_t<8, 8, 1>(a, s);
  return fail(DSPARK_ERR_SHAPE, "moe: no per-CU gate/up instance for K=%ld", K);
}

}  // namespace dspark

using namespace dspark;

extern "C" int dspark_moe_packed_plan(int64_t M, int64_t H, int64_t I, int64_t E, int64_t k, int bits,
                                     int32_t* out) {
  if (!out) return fail(DSPARK_ERR_ARG, "moe_packed_plan: null pointer");
  out[0] = moe_cu_gate_up(M, H, I, E, k, bits) ? 1 : 0;
  out[1] = 0;  // down: one workgroup per (expert, strip) (a per-CU down measured no faster)
  return DSPARK_OK;
}
