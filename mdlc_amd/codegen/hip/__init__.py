"""The HIP backend: templates, lowering, hipRTC runtime and executor."""

from mdlc_amd.codegen.hip.emit import HipCodegen, HipModule, Launch, emit_hip_module

__all__ = ["HipCodegen", "HipModule", "Launch", "emit_hip_module"]
