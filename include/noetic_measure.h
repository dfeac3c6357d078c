/*
 * noetic_measure.h — platform figures that bench.py reports beside the roofline.
 *
 * No counterpart in the reference: the benchmark's roofline compares the fused kernels with the
 * nominal HBM peak, and these two measurements, taken with the library's own kernels on its
 * stream, give the practical floor of one launch on the box that runs it:
 *  - the streaming-read rate of the device (a plain read of `bytes`, a multiple of 128 MiB larger
 *    than the 256 MB Infinity Cache, repeated `reps` times; GB/s = bytes x reps / HIP-event time);
 *  - the period of back-to-back dependent launches of a kernel that does nothing, with the
 *    grid and block shape the caller names (us per launch over `launches` launches);
 *  - the shader clock under a load of dependent fused multiply-adds on every SIMD, held for
 *    `seconds_ms` (the clock settles over the first tenths of a second): the median over the
 *    blocks of the last launch of shader-clock cycles per 10 ns real-time tick, in MHz. The
 *    Gumbel sampler's VALU roofline is priced at this clock.
 * Both need a claimed device (nt_hip_claim) and run on the library stream.
 */
#ifndef NOETIC_MEASURE_H
#define NOETIC_MEASURE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int nt_measure_read(size_t bytes, int32_t reps, double *gbs);
int nt_measure_launch_period(int32_t blocks, int32_t threads, int32_t launches, double *us);
int nt_measure_shader_clock(int32_t seconds_ms, double *mhz);

#ifdef __cplusplus
}
#endif
#endif
