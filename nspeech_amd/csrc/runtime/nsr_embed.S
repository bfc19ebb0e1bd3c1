/* Embeds the gfx950 code objects (one per kernel unit, built into the
 * directory NSR_CO_DIR) into libnspeech_rocm.so's read-only data; the runtime
 * loads each with hipModuleLoadData. The unit list matches
 * nspeech_amd/build.py UNITS and kUnits in nsr_runtime.cpp. */
#define NSR_STR2(x) #x
#define NSR_STR(x) NSR_STR2(x)
#define NSR_EMBED(unit)                                           \
    .section .rodata.nsr_co_##unit, "a", @progbits;                \
    .p2align 12;                                                  \
    .global nsr_co_##unit;                                        \
    .type nsr_co_##unit, @object;                                 \
nsr_co_##unit:;                                                   \
    .incbin NSR_STR(NSR_CO_DIR/nsr_##unit##_gfx950.hsaco);         \
    .byte 0

NSR_EMBED(q8_0_gather)
NSR_EMBED(layernorm)
NSR_EMBED(rotary)
NSR_EMBED(adain_snake)
NSR_EMBED(elementwise)
NSR_EMBED(gemv_q8)
NSR_EMBED(conv1d)
NSR_EMBED(attention)
NSR_EMBED(istft)
NSR_EMBED(calib)

    .section .note.GNU-stack, "", @progbits
