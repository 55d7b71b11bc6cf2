/*
 * pjrtx_custom_call.h — custom-call target registration, under the
 * reference's own export names (reference: src/plugin/custom_call.zig:
 * 158-185, exported from libpjrtx_metal_plugin.dylib and called by its
 * ctypes smoke, src/plugin/pjrt/plugin_ctypes_smoke.py:105-171).
 *
 * A stablehlo.custom_call whose call_target_name is registered lowers to
 * the elementwise op the registration names and fuses like that op (the
 * reference: src/backend/mlx_metal/custom_call.zig:155-238,
 * lowering_custom_call.zig:17-215):
 *   identity  one input, one output of the same dtype and shape;
 *   unary     negate exp expm1 tanh sqrt rsqrt abs cbrt ceil floor log log1p
 *             logistic sine cosine not sign is_finite round_nearest_afz
 *             round_nearest_even popcnt count_leading_zeros;
 *   binary    add subtract multiply divide maximum minimum power atan2
 *             remainder and or xor shift_left shift_right_logical
 *             shift_right_arithmetic (two inputs and the output of one
 *             dtype and shape).
 * Built-in targets: "annotate_device_placement" (identity) and
 * "pjrtx.mlx_metal.custom_binary_add_f32" (add of f32 tensors); the
 * scaled-dot-product-attention target is described in INTEGRATION.md.
 *
 * The registry is process-wide and versioned: a registration change makes
 * later compiles miss the executable cache. Registration returns null on
 * success or a PJRT_Error (INVALID_ARGUMENT: null or empty target, unknown op
 * name), to be read and destroyed through the PJRT_Api error functions.
 *
 * The same registrations are reachable through the PJRT GPU custom-call
 * extension (PJRT_Api.extension_start, pjrt_c_api.h), whose handler_execute
 * must be one of the marker functions below.
 */
#ifndef PJRTX_AMD_PJRTX_CUSTOM_CALL_H_
#define PJRTX_AMD_PJRTX_CUSTOM_CALL_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PJRTX_CC_API __attribute__((visibility("default")))

struct PJRT_Error;

/* Replaces PjRTx_RegisterCustomCallIdentity (custom_call.zig:158-161). */
PJRTX_CC_API struct PJRT_Error* PjRTx_RegisterCustomCallIdentity(const char* function_name,
                                                                 size_t function_name_size);
/* Replaces PjRTx_RegisterCustomCallUnary (custom_call.zig:163-166). */
PJRTX_CC_API struct PJRT_Error* PjRTx_RegisterCustomCallUnary(const char* function_name, size_t function_name_size,
                                                              const char* op_name, size_t op_name_size);
/* Replaces PjRTx_RegisterCustomCallBinary (custom_call.zig:168-171). */
PJRTX_CC_API struct PJRT_Error* PjRTx_RegisterCustomCallBinary(const char* function_name, size_t function_name_size,
                                                               const char* op_name, size_t op_name_size);
/* Replaces PjRTx_UnregisterCustomCall (custom_call.zig:182-185). Built-in
 * targets and unknown names are left alone. */
PJRTX_CC_API void PjRTx_UnregisterCustomCall(const char* function_name, size_t function_name_size);

/* Marker handlers for the PJRT GPU custom-call extension: registering one of
 * these addresses as handler_execute registers an identity, a sqrt or an add
 * target (custom_call.zig:173-180). They are never called. */
PJRTX_CC_API void PjRTx_CustomCall_Identity(void);
PJRTX_CC_API void PjRTx_CustomCall_UnarySqrt(void);
PJRTX_CC_API void PjRTx_CustomCall_BinaryAdd(void);

#ifdef __cplusplus
}
#endif

#endif /* PJRTX_AMD_PJRTX_CUSTOM_CALL_H_ */
