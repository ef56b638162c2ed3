"""Graph passes producing the fused groups the HIP backend consumes."""

from mdlc_amd.passes.base import Pass, PassManager, default_pipeline
from mdlc_amd.passes.constant_folding import ConstantFolding
from mdlc_amd.passes.dce import DeadCodeElimination
from mdlc_amd.passes.fuse_conv_bn import FuseConvBN
from mdlc_amd.passes.fuse_activation import FuseActivation
from mdlc_amd.passes.fuse_elementwise import FuseElementwise

__all__ = ["Pass", "PassManager", "default_pipeline", "ConstantFolding",
           "DeadCodeElimination", "FuseConvBN", "FuseActivation", "FuseElementwise"]
