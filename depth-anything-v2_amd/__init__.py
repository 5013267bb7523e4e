"""ctypes binding of libdepth_anything_v2.so (the MI355X build).

The package directory name is not a Python identifier; load it by path:

    spec = importlib.util.spec_from_file_location("dav2_amd", "<repo>/depth-anything-v2_amd/__init__.py")

`load()` returns the shared library with every entry point of
include/depth_anything_v2.h, include/dav2_hip.h and include/dav2_ops.h
prototyped. There is no fallback: a missing library raises.
"""

from __future__ import annotations

import ctypes as C
import importlib.util
import os
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = PACKAGE_DIR / "libdepth_anything_v2.so"

_lib = None


def _load_sibling(name: str):
    import sys
    key = f"dav2_amd_{name}"
    if key in sys.modules:
        return sys.modules[key]
    spec = importlib.util.spec_from_file_location(key, PACKAGE_DIR / f"{name}.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[key] = mod
    spec.loader.exec_module(mod)
    return mod


dav2_format = _load_sibling("dav2_format")

# ---- ABI types (include/depth_anything_v2.h) ----------------------------------
DAV2_ABI_VERSION = 1
STATUS = {0: "OK", 1: "INVALID_ARGUMENT", 2: "MODEL_IO", 3: "MODEL_FORMAT", 4: "VULKAN_UNAVAILABLE",
          5: "OUT_OF_MEMORY", 6: "INFERENCE_FAILED", 7: "BUFFER_TOO_SMALL", 8: "UNSUPPORTED",
          9: "INTERNAL_ERROR", 10: "INVALID_STATE", 11: "CANCELLED"}
FORCE_FP32, FORCE_FP32_WEIGHTS, FORCE_FP32_ATTENTION, FORCE_FP16, FORCE_INT8, FORCE_METAL, FORCE_VULKAN = (
    1, 2, 4, 8, 16, 32, 64)
REFERENCE_FP16_ATTENTION = 1 << 16  # extension: the reference's binary16 attention in int8 mode
REFERENCE_FP16_COOP_ATTENTION = 1 << 17  # extension: the same with the cooperative-matrix score shader
ENCODER = {"vits": 0, "vitb": 1, "vitl": 2}
GEMM_EPI = {"raw": 0, "row": 1, "row_gelu": 2, "row_layerscale": 3, "transposed": 4, "convt": 5}


class CreateOptions(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32), ("encoder", C.c_int),
                ("vulkan_device_index", C.c_int32), ("flags", C.c_uint32), ("cache_path_utf8", C.c_char_p)]


class ModelInfo(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32), ("encoder", C.c_int),
                ("is_metric", C.c_uint32), ("metric_max_depth", C.c_float), ("reserved", C.c_uint32 * 3)]


class ImageShape(C.Structure):
    _fields_ = [("width", C.c_int32), ("height", C.c_int32)]


class GpuCapabilities(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32), ("flags", C.c_uint64),
                ("adapter_luid", C.c_uint64), ("maximum_in_flight_jobs", C.c_uint32), ("reserved", C.c_uint32)]


class TransferCounters(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("reserved", C.c_uint32), ("tensor_upload_bytes", C.c_uint64),
                ("tensor_download_bytes", C.c_uint64)]


class D3D12TextureSubmitRequest(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32), ("shared_texture_handle", C.c_uint64),
                ("width", C.c_uint32), ("height", C.c_uint32), ("pixel_format", C.c_uint32),
                ("input_size", C.c_int32), ("wait_fence_handle", C.c_uint64), ("wait_fence_value", C.c_uint64),
                ("source_frame_id", C.c_uint64), ("timestamp_ns", C.c_uint64)]


class DeviceBuffer(C.Structure):
    _fields_ = [("data", C.c_void_p), ("bytes", C.c_uint64)]


class GemmArgs(C.Structure):
    _fields_ = [("a", C.c_void_p), ("lda", C.c_uint64), ("b", C.c_void_p), ("ldb", C.c_uint64),
                ("m", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32), ("epilogue", C.c_uint32),
                ("a_scales", C.c_void_p), ("b_scales", C.c_void_p), ("bias", C.c_void_p),
                ("out_i32", C.c_void_p), ("out", C.c_void_p), ("out_row_offset", C.c_uint64),
                ("out_row_stride", C.c_uint64), ("residual", C.c_void_p), ("gamma", C.c_void_p),
                ("convt_kernel", C.c_uint32), ("convt_width", C.c_uint32), ("convt_height", C.c_uint32),
                ("convt_channels", C.c_uint32), ("col_absmax", C.c_void_p), ("col_absmax_begin", C.c_uint32),
                ("relu_output", C.c_uint32), ("split_k", C.c_uint32), ("split_scratch", C.c_void_p)]


class HipSubmitRequest(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("abi_version", C.c_uint32), ("input", C.c_void_p),
                ("input_byte_size", C.c_uint64), ("width", C.c_uint32), ("height", C.c_uint32),
                ("row_stride_bytes", C.c_uint32), ("pixel_format", C.c_uint32), ("input_size", C.c_int32),
                ("flags", C.c_uint32), ("wait_event", C.c_void_p), ("output", C.c_void_p),
                ("output_byte_size", C.c_uint64), ("input_offset", C.c_uint64), ("output_offset", C.c_uint64),
                ("input_ipc", C.c_uint8 * 64), ("output_ipc", C.c_uint8 * 64), ("wait_event_ipc", C.c_uint8 * 64),
                ("source_frame_id", C.c_uint64), ("timestamp_ns", C.c_uint64)]


class GpuJobStatus(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("state", C.c_uint32), ("output_count", C.c_uint32),
                ("reserved", C.c_uint32), ("source_frame_id", C.c_uint64)]


GPU_PIXEL_BGRA8, GPU_PIXEL_RGBA8 = 1, 2
GPU_JOB_QUEUED, GPU_JOB_RUNNING, GPU_JOB_COMPLETE, GPU_JOB_FAILED, GPU_JOB_CANCELLED = 0, 1, 2, 3, 4
HIP_SUBMIT_WAIT_EVENT_IPC = 1


class GemmF32Args(C.Structure):
    _fields_ = [("a", C.c_void_p), ("lda", C.c_uint64), ("b", C.c_void_p), ("ldb", C.c_uint64),
                ("m", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32), ("epilogue", C.c_uint32),
                ("bias", C.c_void_p), ("out", C.c_void_p), ("out_row_offset", C.c_uint64),
                ("out_row_stride", C.c_uint64), ("residual", C.c_void_p), ("gamma", C.c_void_p),
                ("convt_kernel", C.c_uint32), ("convt_width", C.c_uint32), ("convt_height", C.c_uint32),
                ("convt_channels", C.c_uint32), ("relu_output", C.c_uint32), ("half_operands", C.c_uint32)]


class ConvArgs(C.Structure):
    _fields_ = [("input", C.c_void_p), ("width", C.c_uint32), ("height", C.c_uint32), ("channels", C.c_uint32),
                ("kernel", C.c_uint32), ("weight", C.c_void_p), ("weight_scales", C.c_void_p), ("bias", C.c_void_p),
                ("out_channels", C.c_uint32), ("out", C.c_void_p), ("scratch", C.c_void_p),
                ("scratch_floats", C.c_uint64), ("flags", C.c_uint32), ("residual", C.c_void_p),
                ("partial_in", C.c_void_p), ("partial_out", C.c_void_p)]


CONV_RELU_INPUT, CONV_RELU_OUTPUT, CONV_EMIT_ABSMAX, CONV_EMIT_RELU_MAX = 1, 2, 4, 8


vp, u32, i32, u64, f32, sz = C.c_void_p, C.c_uint32, C.c_int32, C.c_uint64, C.c_float, C.c_size_t
DB = DeviceBuffer

# name -> (restype, argtypes)
PROTOTYPES = {
    # public ABI
    "dav2_abi_version": (u32, []),
    "dav2_version_string": (C.c_char_p, []),
    "dav2_status_string": (C.c_char_p, [C.c_int]),
    "dav2_last_error": (C.c_char_p, []),
    "dav2_get_network_shape": (C.c_int, [i32, i32, i32, C.POINTER(ImageShape)]),
    "dav2_get_inferbridge_shape": (C.c_int, [i32, i32, i32, C.POINTER(ImageShape)]),
    "dav2_create": (C.c_int, [C.c_char_p, C.POINTER(CreateOptions), C.POINTER(vp)]),
    "dav2_get_model_info": (C.c_int, [vp, C.POINTER(ModelInfo)]),
    "dav2_prepare": (C.c_int, [vp, i32, i32, i32]),
    "dav2_destroy": (None, [vp]),
    "dav2_probe_gpu_capabilities": (C.c_int, [i32, C.POINTER(GpuCapabilities)]),
    "dav2_get_gpu_capabilities": (C.c_int, [vp, C.POINTER(GpuCapabilities)]),
    "dav2_get_transfer_counters": (C.c_int, [vp, C.POINTER(TransferCounters)]),
    "dav2_submit_d3d12": (C.c_int, [vp, vp, C.POINTER(vp)]),
    "dav2_submit_d3d12_texture": (C.c_int, [vp, C.POINTER(D3D12TextureSubmitRequest), C.POINTER(vp)]),
    "dav2_submit_d3d12_texture_binding": (C.c_int, [vp, vp, C.POINTER(vp)]),
    "dav2_submit_metal_texture_binding": (C.c_int, [vp, vp, C.POINTER(vp)]),
    "dav2_gpu_job_poll": (C.c_int, [vp, vp]),
    "dav2_submit_hip": (C.c_int, [vp, vp, C.POINTER(C.c_void_p)]),
    "dav2_gpu_job_cancel": (C.c_int, [vp]),
    "dav2_gpu_job_release": (None, [vp]),
    "dav2_gpu_output_acquire": (C.c_int, [vp, u32, vp, C.POINTER(vp)]),
    "dav2_gpu_texture_output_acquire": (C.c_int, [vp, u32, vp, C.POINTER(vp)]),
    "dav2_gpu_output_release": (None, [vp]),
    "dav2_infer_bgr8": (C.c_int, [vp, vp, i32, i32, C.c_ssize_t, i32, vp, sz]),
    "dav2_inferbridge_bgra8_f32": (C.c_int, [vp, vp, i32, i32, C.c_ssize_t, i32, vp, sz]),
    "dav2_infer_tensor_f32": (C.c_int, [vp, vp, i32, i32, vp, sz]),
    "dav2_infer_tensor_f32_device": (C.c_int, [vp, vp, i32, i32, i32, vp, sz, vp]),
    "dav2_normalize_relative_device": (C.c_int, [vp, vp, sz, vp]),
    "dav2_profile_enable": (C.c_int, [vp, i32]),
    "dav2_profile_report": (C.c_int, [vp, C.c_char_p, sz]),
    # HIP launcher layer
    "dav2_hip_quantize_rows_i8": (C.c_int, [vp, u64, u32, u32, vp, u32, vp, vp]),
    "dav2_hip_gelu_quantize_rows_i8": (C.c_int, [vp, u64, u32, u32, vp, u32, vp, vp]),
    "dav2_hip_im2col_scratch_floats": (u64, [u32, u32, u32]),
    "dav2_hip_im2col_quantize_i8": (C.c_int, [vp, u32, u32, u32, u32, u32, u32, u32, i32, vp, u32, vp, vp, u64, vp]),
    "dav2_hip_im2col_quantize_relu_i8": (C.c_int, [vp, u32, u32, u32, u32, u32, u32, u32, i32, vp, u32, vp, vp, u64, vp]),
    "dav2_hip_conv2d_i8_supported": (C.c_int, [u32, u32, u32, u32, u32, u32, u32]),
    "dav2_hip_conv_weights_pack": (C.c_int, [vp, vp, u32, u32, u32, u64, vp]),
    "dav2_hip_conv2d_i8": (C.c_int, [C.POINTER(ConvArgs), vp]),
    "dav2_hip_conv1x1_narrow_i8": (C.c_int, [vp, u32, u32, u32, vp, u32, vp, vp, u32, vp, vp, u32, vp]),
    "dav2_hip_layer_norm": (C.c_int, [vp, vp, vp, vp, u32, u32, f32, vp]),
    "dav2_hip_layer_norm_quantize_i8": (C.c_int, [vp, u32, vp, vp, vp, vp, vp, u32, u32, f32, vp]),
    "dav2_hip_gemm_i8": (C.c_int, [C.POINTER(GemmArgs), vp]),
    "dav2_hip_gemm_i8_row_tiles": (u32, [u32, u32, u32]),
    "dav2_hip_gemm_i8_split_scratch_bytes": (u64, [u32, u32, u32]),
    "dav2_hip_gelu": (C.c_int, [vp, vp, u64, vp]),
    "dav2_hip_add_scaled": (C.c_int, [vp, vp, vp, vp, u64, u32, vp]),
    "dav2_hip_add": (C.c_int, [vp, vp, vp, u64, vp]),
    "dav2_hip_relu": (C.c_int, [vp, vp, u64, vp]),
    "dav2_hip_round_half": (C.c_int, [vp, u64, vp]),
    "dav2_hip_attention_scores": (C.c_int, [vp, vp, u32, u32, u32, C.c_int, vp]),
    "dav2_hip_softmax_rows": (C.c_int, [vp, u64, u32, u32, C.c_int, vp]),
    "dav2_hip_attention_values": (C.c_int, [vp, vp, vp, u32, u32, u32, C.c_int, vp]),
    "dav2_hip_attention_scratch_bytes": (u64, [u32, u32, u32, C.c_int]),
    "dav2_hip_attention_ref_scratch_bytes": (u64, [u32, u32, u32, C.c_int]),
    "dav2_hip_pad_rows_i8": (C.c_int, [vp, u32, u32, vp, u32, vp]),
    "dav2_hip_attention_ref_scores": (C.c_int, [vp, vp, u32, u32, u32, C.c_int, vp]),
    "dav2_hip_attention_ref_softmax": (C.c_int, [vp, u64, u32, C.c_int, vp]),
    "dav2_hip_attention_ref_values": (C.c_int, [vp, vp, vp, u32, u32, u32, C.c_int, vp]),
    "dav2_hip_attention_ref16_fused_scratch_bytes": (u64, [u32, u32, u32]),
    "dav2_hip_attention_ref16_fused": (C.c_int, [vp, vp, u32, u32, u32, vp, u64, vp]),
    "dav2_hip_attention_ref16_fused_coop": (C.c_int, [vp, vp, u32, u32, u32, vp, u64, vp]),
    "dav2_hip_attention_ref_scores_coop": (C.c_int, [vp, vp, u32, u32, u32, vp]),
    "dav2_hip_transpose_rows_i8": (C.c_int, [vp, u32, u32, vp, u32, vp]),
    "dav2_hip_attention_fused_scratch_bytes": (u64, [u32, u32, u32]),
    "dav2_hip_attention_fused": (C.c_int, [vp, vp, u32, u32, u32, vp, u64, vp]),
    "dav2_hip_attention_fused_colmax": (C.c_int, [vp, vp, u32, u32, vp, u32, vp, u64, vp]),
    "dav2_hip_bilinear_align_true": (C.c_int, [vp, vp, u32, u32, u32, u32, u32, vp]),
    "dav2_hip_bilinear_align_true_maxima": (C.c_int, [vp, vp, vp, u32, u32, u32, u32, u32, vp]),
    "dav2_hip_conv2d_i8_emits": (C.c_int, [u32, u32]),
    "dav2_hip_gemm_i8_events": (None, [vp, vp]),
    "dav2_hip_launch_events": (C.c_int, [vp, vp]),
    "dav2_hip_minmax_partials": (u32, [u64]),
    "dav2_hip_reduce_minmax": (C.c_int, [vp, u64, vp, vp, vp]),
    "dav2_hip_normalize_relative": (C.c_int, [vp, vp, u64, vp]),
    "dav2_hip_gemm_f32": (C.c_int, [C.c_void_p, vp]),
    "dav2_hip_gemm_h16_products": (C.c_int, [C.c_void_p, vp]),
    "dav2_hip_im2col_f32": (C.c_int, [vp, u32, u32, u32, u32, u32, u32, u32, i32, u32, vp, u32, vp]),
    "dav2_hip_preprocess_bgr8": (C.c_int, [vp, u32, u32, u64, u32, u32, vp, vp]),
    "dav2_hip_preprocess_bgra8_nearest": (C.c_int, [vp, u32, u32, u64, u32, u32, vp, vp]),
    "dav2_hip_normalize_span": (C.c_int, [vp, vp, u64, vp, vp]),
    "dav2_hip_preprocess_rgba8": (C.c_int, [vp, u32, u32, u64, u32, u32, u32, vp, vp]),
    "dav2_hip_position_bicubic": (C.c_int, [vp, vp, u32, u32, u32, vp]),
    "dav2_hip_finish_tokens": (C.c_int, [vp, vp, vp, vp, u32, u32, u32, u32, vp]),
    "dav2_hip_error_string": (C.c_char_p, [C.c_int]),
    # operator surface
    "dav2_ops_create": (vp, [i32]),
    "dav2_ops_destroy": (None, [vp]),
    "dav2_ops_last_error": (C.c_char_p, []),
    "dav2_ops_stream": (vp, [vp]),
    "dav2_ops_synchronize": (C.c_int, [vp]),
    "dav2_ops_linear_int8": (C.c_int, [vp, DB, DB, DB, DB, DB, u32, u32, u32, i32, i32]),
    "dav2_ops_linear_int8_noalloc": (C.c_int, [vp, DB, DB, DB, DB, DB, u32, u32, u32, i32, i32]),
    "dav2_ops_layer_norm": (C.c_int, [vp, DB, DB, DB, DB, u32, u32, f32]),
    "dav2_ops_add_scaled": (C.c_int, [vp, DB, DB, DB, DB, u32, u32]),
    "dav2_ops_attention_head64": (C.c_int, [vp, DB, DB, u32, u32, DB, i32]),
    "dav2_ops_prepare_tokens": (C.c_int, [vp, DB, DB, DB, DB, DB, DB, DB, u32, u32, u32]),
    "dav2_ops_project_tokens_int8": (C.c_int, [vp, DB, DB, DB, DB, DB, u32, u32, u32, u32]),
    "dav2_ops_conv2d_int8": (C.c_int, [vp, DB, DB, DB, DB, DB, u32, u32, u32, u32, u32, u32, u32, i32]),
    "dav2_ops_conv_transpose_nonoverlap_int8": (C.c_int, [vp, DB, DB, DB, DB, DB, u32, u32, u32, u32, u32]),
    "dav2_ops_linear": (C.c_int, [vp, DB, DB, DB, DB, u32, u32, u32, i32]),
    "dav2_ops_project_tokens": (C.c_int, [vp, DB, DB, DB, DB, u32, u32, u32, u32]),
    "dav2_ops_conv2d": (C.c_int, [vp, DB, DB, DB, DB, u32, u32, u32, u32, u32, u32, u32, i32]),
    "dav2_ops_conv_transpose_nonoverlap": (C.c_int, [vp, DB, DB, DB, DB, u32, u32, u32, u32, u32]),
    "dav2_ops_prepare_tokens_f32": (C.c_int, [vp, DB, DB, DB, DB, DB, DB, u32, u32, u32]),
    "dav2_ops_bilinear_align_true": (C.c_int, [vp, DB, DB, u32, u32, u32, u32, u32]),
    "dav2_ops_reduce_minmax": (C.c_int, [vp, DB, DB, u32]),
    "dav2_ops_normalize_relative": (C.c_int, [vp, DB, DB, u32]),
    "dav2_ops_relu": (C.c_int, [vp, DB, DB, u32]),
    "dav2_ops_add": (C.c_int, [vp, DB, DB, DB, u32]),
    "dav2_ops_gelu": (C.c_int, [vp, DB, DB, u32]),
    "dav2_infer_tensor_f32_device_logits": (C.c_int, [vp, vp, i32, i32, vp, vp, vp]),
}


def load(path: str | os.PathLike | None = None):
    """Loads and prototypes the library; raises if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIBRARY_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} is not built (run __graft_entry__.build() or make -C csrc)")
    lib = C.CDLL(str(p))
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(status: int, lib=None) -> None:
    if status != 0:
        lib = lib or load()
        msg = (lib.dav2_last_error() or b"").decode() or (lib.dav2_ops_last_error() or b"").decode()
        raise RuntimeError(f"dav2 status {STATUS.get(status, status)}: {msg}")


def create_options(encoder: str, flags: int = FORCE_INT8, device: int = 0) -> CreateOptions:
    return CreateOptions(C.sizeof(CreateOptions), DAV2_ABI_VERSION, ENCODER[encoder], device, flags, None)


class Context:
    """Owning wrapper of a dav2_context (create -> infer -> destroy)."""

    def __init__(self, model_path: str, encoder: str, flags: int = FORCE_INT8, device: int = 0):
        self.lib = load()
        self.handle = vp()
        opts = create_options(encoder, flags, device)
        check(self.lib.dav2_create(str(model_path).encode(), C.byref(opts), C.byref(self.handle)), self.lib)

    def close(self) -> None:
        if self.handle:
            self.lib.dav2_destroy(self.handle)
            self.handle = vp()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def infer(self, chw, width: int, height: int):
        import numpy as np
        x = np.ascontiguousarray(chw, dtype=np.float32)
        out = np.empty(width * height, dtype=np.float32)
        check(self.lib.dav2_infer_tensor_f32(self.handle, x.ctypes.data, width, height, out.ctypes.data, out.size),
              self.lib)
        return out.reshape(height, width)

    def infer_bgr8(self, image, input_size: int = 518):
        """image: uint8 [H][W][3] BGR (cv2.imread order); returns float32 [H][W] depth."""
        import numpy as np
        img = np.ascontiguousarray(image, dtype=np.uint8)
        height, width = img.shape[0], img.shape[1]
        return self.infer_bgr8_rows(img, width, height, width * 3, input_size)

    def infer_bgr8_rows(self, buf, width: int, height: int, stride: int, input_size: int = 518):
        """buf: uint8 buffer of `height` rows, `stride` bytes apart, 3 bytes per pixel."""
        import numpy as np
        buf = np.ascontiguousarray(buf, dtype=np.uint8)
        out = np.empty(max(width, 0) * max(height, 0), dtype=np.float32)
        check(self.lib.dav2_infer_bgr8(self.handle, buf.ctypes.data, width, height, stride, input_size,
                                       out.ctypes.data, out.size), self.lib)
        return out.reshape(height, width)

    def inferbridge_bgra8(self, image, input_size: int = 518):
        """image: uint8 [H][W][4] BGRA; returns float32 min/max-normalised depth
        at the transposed network shape (dav2_get_inferbridge_shape)."""
        import numpy as np
        img = np.ascontiguousarray(image, dtype=np.uint8)
        height, width = img.shape[0], img.shape[1]
        shape = ImageShape()
        check(self.lib.dav2_get_inferbridge_shape(width, height, input_size, C.byref(shape)), self.lib)
        out = np.empty(shape.width * shape.height, dtype=np.float32)
        check(self.lib.dav2_inferbridge_bgra8_f32(self.handle, img.ctypes.data, width, height, width * 4, input_size,
                                                  out.ctypes.data, out.size), self.lib)
        return out.reshape(shape.height, shape.width)

    def profile(self, enable: bool) -> None:
        check(self.lib.dav2_profile_enable(self.handle, int(enable)), self.lib)

    def profile_report(self) -> dict:
        import json
        buf = C.create_string_buffer(1 << 16)
        check(self.lib.dav2_profile_report(self.handle, buf, len(buf)), self.lib)
        return json.loads(buf.value.decode())

    def infer_device(self, input_ptr: int, batch: int, width: int, height: int, output_ptr: int,
                     output_count: int, stream: int | None = None) -> None:
        check(self.lib.dav2_infer_tensor_f32_device(self.handle, input_ptr, batch, width, height, output_ptr,
                                                    output_count, stream), self.lib)
