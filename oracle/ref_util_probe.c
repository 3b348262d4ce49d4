/*
 * ref_util_probe.c -- exports the reference's own bf16 conversions
 * (c/src/util.h:56-71, compiled from the reference checkout where it lies)
 * so the tests can compare the oracle's restatement against them.
 * TEST INFRASTRUCTURE ONLY; built into oracle/_ref/ by the oracle Makefile.
 */
#include "util.h"

float ref_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }
uint16_t ref_f32_to_bf16(float f) { return f32_to_bf16(f); }
