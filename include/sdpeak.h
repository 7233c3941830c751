/*
 * sdpeak.h - achievable-peak microbenchmarks of the MI355X (gfx950), libsdpeak.so.
 *
 * No counterpart in the reference: these entry points measure the ceilings the benchmark states
 * its kernel-class fractions against, beside the published peaks.  They are used by bench.py
 * (--peak, and the `achievable` fields of its roofline) and touch no engine state.
 *
 * Conventions as in sdhip.h: 0 on success, else nonzero with a NUL-terminated message in err.
 * Each call allocates what it needs, runs one warm-up launch and then `launches` back-to-back
 * launches between two HIP events on `stream` (null: the default stream), and returns
 * out[0] = ms of all timed launches, out[1] = the rate, out[2] = the mean shader clock (GHz) of the
 * last launch's workgroups (s_memtime against the 100 MHz s_memrealtime), out[3] = compute units.
 */
#ifndef SDPEAK_H
#define SDPEAK_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* MFMA loops, wg_per_cu workgroups of 4 waves per compute unit, `iters` loop trips per wave;
 * out[1] in TFLOP/s (f16, 2 flops per multiply-add).
 *  variant 0: v_mfma_f32_32x32x16_f16 alone, 4 independent accumulators per wave;
 *  variant 1: the prefill GEMM's (2,1) inner loop without memory traffic: per 16-k slice one int4
 *             word dequantized as the GEMM does, 2 A fragments from LDS, 2 MFMAs;
 *  variant 2: the same with 4 A fragments and 4 MFMAs per dequantized word (the (4,1) tiles);
 *  variants 3, 4, 5: variants 0, 1, 2 on realistic operands: random f16 signs and mantissas at
 *             magnitudes 2^-3 to 1 (an RMSNorm output's), four operand sets taken in turn so that
 *             consecutive MFMAs see different bits, a random scale per k slice.  MI355X's clock is
 *             power-limited under MFMA load and the power grows with the operand bits that switch:
 *             variants 0-2 (patterned operands, few switching bits) give the instruction-rate
 *             ceiling, variants 3-5 the ceiling a GEMM on real data can reach. */
int sd_peak_mfma(int variant, int wg_per_cu, int iters, int launches, void* stream, double* out, char* err,
                 size_t errlen);

/* HBM streaming over `bytes` (at least 1 MiB, a multiple of 16); out[1] in GB/s of bytes moved.
 *  variant 0: read only; variant 1: copy (read + write counted). */
int sd_peak_hbm(int variant, size_t bytes, int launches, void* stream, double* out, char* err, size_t errlen);

#ifdef __cplusplus
}
#endif

#endif /* SDPEAK_H */
