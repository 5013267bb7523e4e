"""numpy wrapper of the CPU oracle (oracle/liboracle.so). Test infrastructure only."""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_PATH = ROOT / "oracle" / "liboracle.so"

vp, u32, i32, u64, f32, sz = C.c_void_p, C.c_uint32, C.c_int32, C.c_uint64, C.c_float, C.c_size_t

_PROTO = {
    "orc_set_threads": (C.c_int, [C.c_int]),
    "orc_get_threads": (C.c_int, []),
    "orc_quantize_rows": (None, [vp, u32, u32, u32, vp, vp]),
    "orc_im2col_quantize": (None, [vp, u32, u32, u32, u32, u32, u32, u32, i32, vp, vp]),
    "orc_quantize_weight_rows": (None, [vp, u64, u64, vp, vp]),
    "orc_quantize_convT_weight": (None, [vp, u32, u32, u32, vp, vp]),
    "orc_gemm_i8": (None, [vp, vp, u32, u32, u32, vp]),
    "orc_linear_epilogue": (None, [vp, vp, vp, vp, u32, u32, u32, u32, C.c_int, vp]),
    "orc_linear_int8": (None, [vp, vp, vp, vp, u32, u32, u32, C.c_int, vp]),
    "orc_gelu": (None, [vp, u64, vp]),
    "orc_numerator21": (None, [vp, u64, vp]),
    "orc_numerator21_x8": (None, [vp, u64, vp]),
    "orc_exp": (None, [vp, u64, vp]),
    "orc_round_half_product": (None, [vp, vp, u64, vp]),
    "orc_attention_scores_binary16": (None, [vp, u32, u32, vp]),
    "orc_attention_scores_coop": (None, [vp, u32, u32, vp]),
    "orc_layer_norm": (None, [vp, vp, vp, u32, u32, f32, vp]),
    "orc_add_scaled": (None, [vp, vp, vp, u64, u32, vp]),
    "orc_add": (None, [vp, vp, u64, vp]),
    "orc_relu": (None, [vp, u64, vp]),
    "orc_softmax_rows": (None, [vp, u64, u32, vp]),
    "orc_attention_head64": (None, [vp, u32, u32, C.c_int, vp, vp]),
    "orc_bilinear_align_true": (None, [vp, u32, u32, u32, u32, u32, vp]),
    "orc_reduce_minmax": (None, [vp, u64, vp]),
    "orc_normalize_relative": (None, [vp, vp, u64]),
    "orc_position_bicubic": (None, [vp, u32, u32, u32, vp]),
    "orc_prepare_tokens_int8": (None, [vp, vp, vp, vp, vp, vp, u32, u32, u32, vp]),
    "orc_project_tokens_int8": (None, [vp, vp, vp, vp, u32, u32, u32, u32, vp]),
    "orc_conv2d_int8": (None, [vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, C.c_int, vp]),
    "orc_conv_transpose_int8": (None, [vp, vp, vp, vp, u32, u32, u32, u32, u32, vp]),
    "orc_model_load": (vp, [C.c_char_p, C.c_int, C.c_char_p, sz]),
    "orc_model_free": (None, [vp]),
    "orc_model_infer": (C.c_int, [vp, vp, u32, u32, C.c_int, vp, vp, vp]),
    "orc_model_encoder_blocks": (C.c_int, [vp, vp, u32, u32, u32, C.c_int]),
    "orc_model_infer_fp32": (C.c_int, [vp, vp, u32, u32, vp, vp, vp]),
    "orc_linear_f32": (None, [vp, vp, vp, u32, u32, u32, C.c_int, vp]),
    "orc_conv2d_f32": (None, [vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, C.c_int, vp]),
    "orc_conv_transpose_f32": (None, [vp, vp, vp, u32, u32, u32, u32, u32, vp]),
    "orc_project_tokens_f32": (None, [vp, vp, vp, u32, u32, u32, u32, vp]),
    "orc_prepare_tokens_f32": (None, [vp, vp, vp, vp, vp, u32, u32, u32, vp]),
    "orc_model_infer_fp16": (C.c_int, [vp, vp, u32, u32, C.c_int, vp, vp, vp]),
    "orc_gemm_h16_products": (None, [vp, u64, vp, u64, u32, u32, u32, vp]),
    "orc_linear_f16": (None, [vp, vp, vp, u32, u32, u32, C.c_int, C.c_int, vp]),
    "orc_project_tokens_f16": (None, [vp, vp, vp, u32, u32, u32, u32, vp]),
    "orc_conv_transpose_f16": (None, [vp, vp, vp, u32, u32, u32, u32, u32, vp]),
    "orc_prepare_tokens_f16": (None, [vp, vp, vp, vp, vp, u32, u32, u32, vp]),
    "orc_network_shape": (C.c_int, [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "orc_preprocess_bgr8": (None, [vp, C.c_int, C.c_int, C.c_int64, C.c_int, C.c_int, vp]),
    "orc_preprocess_bgra8_nearest": (None, [vp, C.c_int, C.c_int, C.c_int64, C.c_int, C.c_int, vp]),
    "orc_normalize_span": (None, [vp, u64, vp]),
    "orc_preprocess_rgba8": (None, [vp, C.c_int, C.c_int, C.c_int64, C.c_int, C.c_int, C.c_int, vp]),
    "orc_float_to_half": (C.c_uint16, [f32]),
    "orc_half_to_float": (f32, [C.c_uint16]),
    "orc_crc32": (C.c_uint32, [vp, sz]),
}


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


class Oracle:
    def __init__(self, path: Path = ORACLE_PATH):
        if not path.exists():
            raise FileNotFoundError(f"{path} not built (make -C oracle)")
        self.lib = C.CDLL(str(path))
        for name, (res, args) in _PROTO.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args

    # --- quantizers -----------------------------------------------------------
    def quantize_rows(self, x: np.ndarray, rows: int | None = None, columns: int | None = None, input_offset: int = 0):
        x = _f32(x)
        if rows is None:
            rows, columns = x.shape
        q = np.empty((rows, columns), np.int8)
        s = np.empty(rows, np.float32)
        self.lib.orc_quantize_rows(x.ctypes.data, rows, columns, input_offset, q.ctypes.data, s.ctypes.data)
        return q, s

    def im2col_quantize(self, img: np.ndarray, kernel: int, stride: int, padding: int):
        img = _f32(img)
        c, h, w = img.shape
        ow = (w + 2 * padding - kernel) // stride + 1
        oh = (h + 2 * padding - kernel) // stride + 1
        k = c * kernel * kernel
        q = np.empty((ow * oh, k), np.int8)
        s = np.empty(ow * oh, np.float32)
        self.lib.orc_im2col_quantize(img.ctypes.data, w, h, c, ow, oh, kernel, stride, padding, q.ctypes.data,
                                     s.ctypes.data)
        return q, s

    def quantize_weight_rows(self, w: np.ndarray):
        w = _f32(w)
        rows = w.shape[0]
        cols = w.size // rows
        q = np.empty((rows, cols), np.int8)
        s = np.empty(rows, np.float32)
        self.lib.orc_quantize_weight_rows(w.ctypes.data, rows, cols, q.ctypes.data, s.ctypes.data)
        return q, s

    def quantize_convT_weight(self, w: np.ndarray):
        w = _f32(w)
        ic, oc, k, _ = w.shape
        q = np.empty((k * k * oc, ic), np.int8)
        s = np.empty(k * k * oc, np.float32)
        self.lib.orc_quantize_convT_weight(w.ctypes.data, ic, oc, k, q.ctypes.data, s.ctypes.data)
        return q, s

    # --- GEMM -----------------------------------------------------------------
    def gemm_i8(self, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(a, np.int8)
        b = np.ascontiguousarray(b, np.int8)
        m, k = a.shape
        n = b.shape[0]
        acc = np.empty((m, n), np.int32)
        self.lib.orc_gemm_i8(a.ctypes.data, b.ctypes.data, m, n, k, acc.ctypes.data)
        return acc

    def linear_epilogue(self, acc, s_in, s_w, bias, out_rows: int, row_offset=0, row_stride=0, transposed=False):
        acc = np.ascontiguousarray(acc, np.int32)
        rows, cols = acc.shape
        s_in, s_w = _f32(s_in), _f32(s_w)
        bias = None if bias is None else _f32(bias)
        out = np.zeros(out_rows * cols, np.float32)
        self.lib.orc_linear_epilogue(acc.ctypes.data, s_in.ctypes.data, s_w.ctypes.data, _p(bias), rows, cols,
                                     row_offset, row_stride, int(transposed), out.ctypes.data)
        return out

    def linear_int8(self, x, wq, ws, bias, gelu=False):
        x, ws, bias = _f32(x), _f32(ws), _f32(bias)
        wq = np.ascontiguousarray(wq, np.int8)
        rows, ic = x.shape
        oc = wq.shape[0]
        out = np.empty((rows, oc), np.float32)
        self.lib.orc_linear_int8(x.ctypes.data, wq.ctypes.data, ws.ctypes.data, bias.ctypes.data, rows, ic, oc,
                                 int(gelu), out.ctypes.data)
        return out

    # --- elementwise / reductions ---------------------------------------------
    def gelu(self, x):
        x = _f32(x)
        out = np.empty_like(x)
        self.lib.orc_gelu(x.ctypes.data, x.size, out.ctypes.data)
        return out

    def numerator21(self, x):
        x = _f32(x)
        out = np.empty_like(x)
        self.lib.orc_numerator21(x.ctypes.data, x.size, out.ctypes.data)
        return out

    def exp(self, x):
        x = _f32(x)
        out = np.empty_like(x)
        self.lib.orc_exp(x.ctypes.data, x.size, out.ctypes.data)
        return out

    def layer_norm(self, x, w, b, eps=1e-6):
        x, w, b = _f32(x), _f32(w), _f32(b)
        out = np.empty_like(x)
        self.lib.orc_layer_norm(x.ctypes.data, w.ctypes.data, b.ctypes.data, x.shape[0], x.shape[1], eps,
                                out.ctypes.data)
        return out

    def add_scaled(self, residual, addend, scale):
        residual, addend, scale = _f32(residual), _f32(addend), _f32(scale)
        out = np.empty_like(residual)
        self.lib.orc_add_scaled(residual.ctypes.data, addend.ctypes.data, scale.ctypes.data, residual.size,
                                scale.size, out.ctypes.data)
        return out

    def add(self, a, b):
        a, b = _f32(a), _f32(b)
        out = np.empty_like(a)
        self.lib.orc_add(a.ctypes.data, b.ctypes.data, a.size, out.ctypes.data)
        return out

    def relu(self, a):
        a = _f32(a)
        out = np.empty_like(a)
        self.lib.orc_relu(a.ctypes.data, a.size, out.ctypes.data)
        return out

    def softmax_rows(self, x):
        x = _f32(x)
        out = np.empty_like(x)
        self.lib.orc_softmax_rows(x.ctypes.data, x.shape[0], x.shape[1], out.ctypes.data)
        return out

    def round_half_product(self, a, b):
        a, b = _f32(a), _f32(b)
        out = np.empty_like(a)
        self.lib.orc_round_half_product(a.ctypes.data, b.ctypes.data, a.size, out.ctypes.data)
        return out

    def scores_binary16(self, qkv, tokens: int, heads: int):
        """Binary16 scores [H][T][T] as float16 (bmm_score_fp16.glsl)."""
        qkv = _f32(qkv)
        out = np.empty((heads, tokens, tokens), np.float16)
        self.lib.orc_attention_scores_binary16(qkv.ctypes.data, tokens, heads, out.ctypes.data)
        return out

    def scores_coop(self, qkv, tokens: int, heads: int):
        """Binary16 scores [H][T][T] as float16 (bmm_score_coop_fp16.glsl: exact
        products summed in double, rounded to fp32, then binary16)."""
        qkv = _f32(qkv)
        out = np.empty((heads, tokens, tokens), np.float16)
        self.lib.orc_attention_scores_coop(qkv.ctypes.data, tokens, heads, out.ctypes.data)
        return out

    def attention(self, qkv, tokens: int, heads: int, fp16: bool = False, probabilities: bool = False,
                  fused: bool = False, coop: bool = False):
        """fp16=False: fp32 path; fp16=True: materialised binary16 scores
        (coop=True: the cooperative-matrix score shader's arithmetic);
        fused=True: the integer-exact kernel of int8 mode."""
        qkv = _f32(qkv)
        out = np.empty((tokens, heads * 64), np.float32)
        p = np.empty((heads, tokens, tokens), np.float32) if probabilities else None
        mode = 2 if fused else (3 if coop else int(fp16))
        self.lib.orc_attention_head64(qkv.ctypes.data, tokens, heads, mode, out.ctypes.data, _p(p))
        return (out, p) if probabilities else out

    def bilinear(self, x, ow: int, oh: int):
        x = _f32(x)
        c, ih, iw = x.shape
        out = np.empty((c, oh, ow), np.float32)
        self.lib.orc_bilinear_align_true(x.ctypes.data, iw, ih, ow, oh, c, out.ctypes.data)
        return out

    def reduce_minmax(self, x):
        x = _f32(x)
        r = np.empty(2, np.float32)
        self.lib.orc_reduce_minmax(x.ctypes.data, x.size, r.ctypes.data)
        return r

    def normalize_relative(self, d, r):
        d = _f32(d).copy()
        r = _f32(r)
        self.lib.orc_normalize_relative(d.ctypes.data, r.ctypes.data, d.size)
        return d

    def network_shape(self, width: int, height: int, input_size: int):
        w, h = C.c_int(), C.c_int()
        if self.lib.orc_network_shape(width, height, input_size, C.byref(w), C.byref(h)) != 0:
            raise ValueError("image dimensions and input_size must be positive")
        return w.value, h.value

    def preprocess_bgr8(self, buf, width: int, height: int, stride: int, dst_width: int, dst_height: int):
        buf = np.ascontiguousarray(buf, dtype=np.uint8)
        assert buf.size >= (height - 1) * stride + 3 * width
        out = np.empty((3, dst_height, dst_width), np.float32)
        self.lib.orc_preprocess_bgr8(buf.ctypes.data, width, height, stride, dst_width, dst_height, out.ctypes.data)
        return out

    def preprocess_bgra8_nearest(self, buf, width: int, height: int, stride: int, dst_width: int, dst_height: int):
        buf = np.ascontiguousarray(buf, dtype=np.uint8)
        assert buf.size >= (height - 1) * stride + 4 * width
        out = np.empty((3, dst_height, dst_width), np.float32)
        self.lib.orc_preprocess_bgra8_nearest(buf.ctypes.data, width, height, stride, dst_width, dst_height,
                                              out.ctypes.data)
        return out

    def preprocess_rgba8(self, words, width: int, height: int, stride_pixels: int, dst_width: int, dst_height: int,
                         rgba: bool):
        """words: uint32 pixels, `height` rows of `stride_pixels`."""
        words = np.ascontiguousarray(words, dtype=np.uint32)
        assert words.size >= (height - 1) * stride_pixels + width
        out = np.empty((3, dst_height, dst_width), np.float32)
        self.lib.orc_preprocess_rgba8(words.ctypes.data, width, height, stride_pixels, dst_width, dst_height, int(rgba),
                                      out.ctypes.data)
        return out

    def normalize_span(self, d):
        d = _f32(d)
        out = np.empty_like(d)
        self.lib.orc_normalize_span(d.ctypes.data, d.size, out.ctypes.data)
        return out

    def position_bicubic(self, position, pw: int, ph: int, dim: int):
        position = _f32(position)
        out = np.empty((dim, ph, pw), np.float32)
        self.lib.orc_position_bicubic(position.ctypes.data, pw, ph, dim, out.ctypes.data)
        return out

    # --- operators ----------------------------------------------------------------
    def prepare_tokens_int8(self, image, wq, ws, bias, cls, pos, width, height, dim):
        image, ws, bias, cls, pos = map(_f32, (image, ws, bias, cls, pos))
        wq = np.ascontiguousarray(wq, np.int8)
        t = (width // 14) * (height // 14) + 1
        out = np.empty((t, dim), np.float32)
        self.lib.orc_prepare_tokens_int8(image.ctypes.data, wq.ctypes.data, ws.ctypes.data, bias.ctypes.data,
                                         cls.ctypes.data, pos.ctypes.data, width, height, dim, out.ctypes.data)
        return out

    def project_tokens_int8(self, tokens, wq, ws, bias, width, height, dim, channels):
        tokens, ws, bias = map(_f32, (tokens, ws, bias))
        wq = np.ascontiguousarray(wq, np.int8)
        out = np.empty((channels, height, width), np.float32)
        self.lib.orc_project_tokens_int8(tokens.ctypes.data, wq.ctypes.data, ws.ctypes.data, bias.ctypes.data,
                                         width, height, dim, channels, out.ctypes.data)
        return out

    def conv2d_int8(self, x, wq, ws, bias, out_channels, kernel, stride, padding, has_bias=True):
        x, ws = _f32(x), _f32(ws)
        bias = _f32(bias) if bias is not None else None
        wq = np.ascontiguousarray(wq, np.int8)
        c, h, w = x.shape
        ow = (w + 2 * padding - kernel) // stride + 1
        oh = (h + 2 * padding - kernel) // stride + 1
        out = np.empty((out_channels, oh, ow), np.float32)
        self.lib.orc_conv2d_int8(x.ctypes.data, wq.ctypes.data, ws.ctypes.data, _p(bias), w, h, c, out_channels,
                                 kernel, stride, padding, int(has_bias), out.ctypes.data)
        return out

    def conv_transpose_int8(self, x, wq, ws, bias, out_channels, kernel):
        x, ws, bias = _f32(x), _f32(ws), _f32(bias)
        wq = np.ascontiguousarray(wq, np.int8)
        c, h, w = x.shape
        out = np.empty((out_channels, h * kernel, w * kernel), np.float32)
        self.lib.orc_conv_transpose_int8(x.ctypes.data, wq.ctypes.data, ws.ctypes.data, bias.ctypes.data, w, h, c,
                                         out_channels, kernel, out.ctypes.data)
        return out

    # --- whole model ---------------------------------------------------------------
    def load_model(self, path, encoder: int):
        err = C.create_string_buffer(256)
        h = self.lib.orc_model_load(str(path).encode(), encoder, err, 256)
        if not h:
            raise RuntimeError(f"oracle could not load {path}: {err.value.decode()}")
        return h

    def free_model(self, h) -> None:
        self.lib.orc_model_free(h)

    def infer_fp32(self, h, chw, width: int, height: int):
        """The graph in the fp32 precision mode; returns (depth, pre-ReLU logits)."""
        chw = _f32(chw)
        depth = np.empty((height, width), np.float32)
        logits = np.empty((height, width), np.float32)
        if self.lib.orc_model_infer_fp32(h, chw.ctypes.data, width, height, depth.ctypes.data, logits.ctypes.data,
                                         None) != 0:
            raise RuntimeError("oracle inference failed")
        return depth, logits

    def linear_f32(self, x, w, b, gelu: bool = False):
        x, w = _f32(x), _f32(w)
        rows, k = x.shape
        n = w.shape[0]
        out = np.empty((rows, n), np.float32)
        self.lib.orc_linear_f32(x.ctypes.data, w.ctypes.data, _p(None if b is None else _f32(b)), rows, k, n,
                                int(gelu), out.ctypes.data)
        return out

    def conv2d_f32(self, x, w, b, stride: int, padding: int):
        x, w = _f32(x), _f32(w)
        ic, ih, iw = x.shape
        oc, _, k, _ = w.shape
        ow, oh = (iw + 2 * padding - k) // stride + 1, (ih + 2 * padding - k) // stride + 1
        out = np.empty((oc, oh, ow), np.float32)
        bb = None if b is None else _f32(b)
        self.lib.orc_conv2d_f32(x.ctypes.data, w.ctypes.data, _p(bb), iw, ih, ic, oc, k, stride, padding,
                                int(b is not None), out.ctypes.data)
        return out

    def conv_transpose_f32(self, x, w, b):
        x, w, b = _f32(x), _f32(w), _f32(b)
        ic, ih, iw = x.shape
        _, oc, k, _ = w.shape
        out = np.empty((oc, ih * k, iw * k), np.float32)
        self.lib.orc_conv_transpose_f32(x.ctypes.data, w.ctypes.data, b.ctypes.data, iw, ih, ic, oc, k,
                                        out.ctypes.data)
        return out

    def project_tokens_f32(self, tokens, w, b, pw: int, ph: int):
        tokens, w, b = _f32(tokens), _f32(w), _f32(b)
        c, d = w.shape
        out = np.empty((c, ph, pw), np.float32)
        self.lib.orc_project_tokens_f32(tokens.ctypes.data, w.ctypes.data, b.ctypes.data, pw, ph, d, c,
                                        out.ctypes.data)
        return out

    def prepare_tokens_f32(self, image, w, b, cls, pos, width: int, height: int):
        image, w, b, cls, pos = _f32(image), _f32(w), _f32(b), _f32(cls), _f32(pos)
        d = w.shape[0]
        t = (width // 14) * (height // 14) + 1
        out = np.empty((t, d), np.float32)
        self.lib.orc_prepare_tokens_f32(image.ctypes.data, w.ctypes.data, b.ctypes.data, cls.ctypes.data,
                                        pos.ctypes.data, width, height, d, out.ctypes.data)
        return out

    # ---- fp16 precision mode ------------------------------------------------
    def infer_fp16(self, h, chw, width: int, height: int, attention: str = "binary16"):
        """The graph in the fp16 precision mode; returns (depth, pre-ReLU logits)."""
        chw = _f32(chw)
        depth = np.empty((height, width), np.float32)
        logits = np.empty((height, width), np.float32)
        if self.lib.orc_model_infer_fp16(h, chw.ctypes.data, width, height, self.ATTENTION_MODES[attention],
                                         depth.ctypes.data, logits.ctypes.data, None) != 0:
            raise RuntimeError("oracle inference failed")
        return depth, logits

    def gemm_h16_products(self, a, b):
        a, b = _f32(a), _f32(b)
        m, k = a.shape
        n = b.shape[0]
        out = np.empty((m, n), np.float32)
        self.lib.orc_gemm_h16_products(a.ctypes.data, k, b.ctypes.data, k, m, n, k, out.ctypes.data)
        return out

    def linear_f16(self, x, w, b, gelu: bool = False, half_output: bool = False):
        x, w = _f32(x), _f32(w)
        rows, k = x.shape
        n = w.shape[0]
        out = np.empty((rows, n), np.float32)
        self.lib.orc_linear_f16(x.ctypes.data, w.ctypes.data, _p(None if b is None else _f32(b)), rows, k, n,
                                int(gelu), int(half_output), out.ctypes.data)
        return out

    def project_tokens_f16(self, tokens, w, b, pw: int, ph: int):
        tokens, w, b = _f32(tokens), _f32(w), _f32(b)
        c, d = w.shape
        out = np.empty((c, ph, pw), np.float32)
        self.lib.orc_project_tokens_f16(tokens.ctypes.data, w.ctypes.data, b.ctypes.data, pw, ph, d, c,
                                        out.ctypes.data)
        return out

    def conv_transpose_f16(self, x, w, b):
        x, w, b = _f32(x), _f32(w), _f32(b)
        ic, ih, iw = x.shape
        _, oc, k, _ = w.shape
        out = np.empty((oc, ih * k, iw * k), np.float32)
        self.lib.orc_conv_transpose_f16(x.ctypes.data, w.ctypes.data, b.ctypes.data, iw, ih, ic, oc, k,
                                        out.ctypes.data)
        return out

    def prepare_tokens_f16(self, image, w, b, cls, pos, width: int, height: int):
        image, w, b, cls, pos = _f32(image), _f32(w), _f32(b), _f32(cls), _f32(pos)
        d = w.shape[0]
        t = (width // 14) * (height // 14) + 1
        out = np.empty((t, d), np.float32)
        self.lib.orc_prepare_tokens_f16(image.ctypes.data, w.ctypes.data, b.ctypes.data, cls.ctypes.data,
                                        pos.ctypes.data, width, height, d, out.ctypes.data)
        return out

    ATTENTION_MODES = {"fp32": 0, "binary16": 1, "exact": 2, "coop": 3}

    def infer(self, h, chw, width: int, height: int, attention: str = "exact", dim: int | None = None):
        """The int8 graph. attention: "exact" (this build's integer-exact
        attention, the int8-mode default of the GPU path; not the reference's
        arithmetic), "binary16" (the reference's int8-mode attention
        arithmetic: bmm_score_fp16 / softmax_lastdim_half / bmm_value_fp16),
        "coop" (the same with bmm_score_coop_fp16's scores) or "fp32"
        (FORCE_FP32_ATTENTION: bmm.glsl / softmax_lastdim.glsl)."""
        mode = self.ATTENTION_MODES[attention]
        chw = _f32(chw)
        depth = np.empty((height, width), np.float32)
        logits = np.empty((height, width), np.float32)
        feats = None
        if dim is not None:
            t = (width // 14) * (height // 14) + 1
            feats = np.empty((4, t, dim), np.float32)
        rc = self.lib.orc_model_infer(h, chw.ctypes.data, width, height, mode, depth.ctypes.data,
                                      logits.ctypes.data, _p(feats))
        if rc != 0:
            raise RuntimeError("oracle inference failed")
        return depth, logits, feats


def pack_conv_weights(q: np.ndarray, n: int, c: int, k: int) -> np.ndarray:
    """int8 conv weights [n][c*k*k] (reference order: c major, then tap) ->
    the implicit convolution's packed layout: K walked tap-major
    (tap * c + ic), cut into 16-row x 64-byte fragments [n/16][K/64], each
    stored lane by lane (lane l: row l % 16, K bytes 16 (l // 16) .. + 15)."""
    taps = k * k
    kk = taps * c
    tm = q[:, :kk].reshape(n, c, taps).transpose(0, 2, 1).reshape(n, kk)
    frags = tm.reshape(n // 16, 16, kk // 64, 4, 16).transpose(0, 2, 3, 1, 4)
    return np.ascontiguousarray(frags).reshape(n, kk)


def pad_rows(q: np.ndarray, ld: int | None = None) -> np.ndarray:
    """int8 [rows][K] -> [rows][ld] with zero padding (the GPU int8 layout)."""
    rows, k = q.shape
    ld = ld or (k + 63) // 64 * 64
    out = np.zeros((rows, ld), np.int8)
    out[:, :k] = q
    return out
