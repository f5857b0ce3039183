// Explicit instantiation of the decode launchers for one (storage type, GQA
// group) pair.  The build compiles this file once per pair with
// -DEKV_INST_DTYPE=<0 fp32 | 1 fp16 | 2 bf16> -DEKV_INST_G=<1 | 2 | 4 | 8>.
#include "decode_launch.h"

#if !defined(EKV_INST_DTYPE) || !defined(EKV_INST_G)
#error "decode_inst.hip is compiled once per (EKV_INST_DTYPE, EKV_INST_G) by entmaxkv_amd/build.py"
#endif

#if EKV_INST_DTYPE == 0
template struct ekv::dec::Launch<float, EKV_INST_G>;
#elif EKV_INST_DTYPE == 1
template struct ekv::dec::Launch<_Float16, EKV_INST_G>;
#else
template struct ekv::dec::Launch<ekv::bf16_t, EKV_INST_G>;
#endif

#ifdef EKV_PHASE_TIMERS
extern "C" int ekv_debug_wave_timers(unsigned long long* host, int n) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(ekv_wave_timers),
                                  n * sizeof(unsigned long long));
}
extern "C" int ekv_debug_phase_timers(unsigned long long* host, int n) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(ekv_phase_timers),
                                  n * sizeof(unsigned long long));
}
#endif
