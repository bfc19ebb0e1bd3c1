/*
 * Unity translation unit: every kernel of the library in one gfx950 code
 * object (built with --genco --no-gpu-bundle-output, embedded in
 * libnspeech_rocm.so and loaded with hipModuleLoadData).
 */
#include "q8_0_gather.hip"
#include "layernorm.hip"
#include "rotary.hip"
#include "adain_snake.hip"
#include "elementwise.hip"
