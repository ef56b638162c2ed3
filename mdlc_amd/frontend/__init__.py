"""ONNX frontend: a protobuf reader and writer for the inference subset of
the ONNX schema, and the importer into the IR (mdlc/frontend/)."""

from mdlc_amd.frontend.onnx_importer import import_onnx, import_onnx_model
from mdlc_amd.frontend.onnx_proto import OnnxDecodeError, load_model, parse_model

__all__ = ["import_onnx", "import_onnx_model", "load_model", "parse_model", "OnnxDecodeError"]
