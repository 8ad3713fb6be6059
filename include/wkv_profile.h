/* Profiling-only entry point of libwkv_phase.so, the library built with
 * WKV_PHASE_CLOCKS (python -m wavelet_amd.build --phase-clocks). Not part of
 * the drop-in ABI of include/wkv.h and not exported by libwkv.so; no
 * reference counterpart.
 *
 * Copies the first n (<= 16384) entries of the MLA decode kernel's per-workgroup
 * phase cycle sums of its latest launch (16 per workgroup, the first 1,024
 * workgroups; slot meanings at kPhaseWgs in wavelet_amd/csrc/decode_mla.hip)
 * to host memory at dst. Synchronous (a hipMemcpyFromSymbol). Returns 0, or
 * WKV_ERR_INVALID / WKV_ERR_LAUNCH. */
#pragma once

#ifdef __cplusplus
extern "C" {
#endif

int wkv_mla_phase_clocks(unsigned long long *dst, int n);

#ifdef __cplusplus
}
#endif
