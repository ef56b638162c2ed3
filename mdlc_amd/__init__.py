"""mdlc_amd — an MI355X-native (gfx950) fused-group backend for the mdlc compiler."""

__version__ = "0.1.0"
