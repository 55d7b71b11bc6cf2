// Custom-call targets: a stablehlo.custom_call whose target is registered
// lowers to the elementwise op the registration names, so it fuses and runs
// like the op itself.
//
// Reference: src/backend/mlx_metal/custom_call.zig:16-102 (registration kinds
// and the unary/binary op-name tables), :155-238 (process registry, version
// counter, built-in targets), src/backend/mlx_metal/lowering_custom_call.zig:
// 17-215 (legality of identity, unary and binary targets), and
// src/plugin/custom_call.zig:1-185 (the PJRT GPU custom-call extension and
// the PjRTx_* exports, in pjrt_api.cc here).
#pragma once

#include <cstdint>
#include <string>

#include "ir.h"

namespace pjrtx {

enum class CustomCallKind { kIdentity, kUnary, kBinary };

struct CustomCallSpec {
  CustomCallKind kind = CustomCallKind::kIdentity;
  OpKind op = OpKind::kParameter;  // kUnary / kBinary: the elementwise op
  bool f32_only = false;           // the built-in f32 add target
};

// Registration (replaces an existing registration of the same target).
// Fails with kInvalidArgument for an empty target or an op name outside the
// tables.
void register_custom_call_identity(const std::string& target);
void register_custom_call_unary(const std::string& target, const std::string& op_name);
void register_custom_call_binary(const std::string& target, const std::string& op_name);
// Removes a registered target; built-in targets and unknown names are left
// alone.
void unregister_custom_call(const std::string& target);

// Built-in targets first ("annotate_device_placement": identity;
// "pjrtx.mlx_metal.custom_binary_add_f32": add of f32 tensors), then the
// registry. The scaled-dot-product-attention target is lowered separately.
bool lookup_custom_call(const std::string& target, CustomCallSpec* spec);

// Counts registry changes; part of the compile-cache key, so an executable
// compiled under one registration is not reused under another.
uint64_t custom_call_registry_version();

// Rewrites a registered custom_call op in place into its elementwise op
// (identity: a reshape to the same shape) after the reference's legality
// checks; kUnimplemented for a target with no registration, kInvalidArgument
// for operands or results that break the target's rules.
void lower_registered_custom_call(const Program& prog, Op* op);

}  // namespace pjrtx
