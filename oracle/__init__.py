"""ctypes front-end of the CPU oracle (oracle/wpc_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker that the HIP library is compared
against, and the CPU baseline that bench.py times. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package; the product (wpc-engine_amd/, include/) never does.

Arrays are numpy; blocks are uint8 arrays in the reference's on-disk byte
layout (68-byte v4 blocks, 100-byte v3 blocks, 132-byte v2 blocks).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

KERNEL_SCALAR, KERNEL_FUSED, KERNEL_AVX2 = 0, 1, 2

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_sz = C.c_size_t


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    args = ["make", "-C", _HERE] + (["-B"] if force else [])
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = C.CDLL(_LIB_PATH)
    sig = {
        "or_f16_to_f32": (C.c_float, [C.c_uint16]),
        "or_f32_to_f16": (C.c_uint16, [C.c_float]),
        "or_f16_to_f32_array": (None, [_u16p, _f32p, _sz]),
        "or_f32_to_f16_array": (None, [_f32p, _u16p, _sz]),
        "or_v4_pack_codes": (None, [_u8p, _u8p]),
        "or_v4_unpack_codes": (None, [_u8p, _u8p]),
        "or_v3_pack_codes": (None, [_u8p, _u8p]),
        "or_v3_unpack_codes": (None, [_u8p, _u8p]),
        "or_v3tp_pack": (None, [_u8p, _u8p, _u8p]),
        "or_v3tp_unpack": (None, [_u8p, _u8p, _u8p]),
        "or_affine_quant_block_v2": (None, [_f32p, _u8p]),
        "or_affine_quant_block_v3": (None, [_f32p, _u8p]),
        "or_affine_quant_block_v4": (None, [_f32p, _u8p]),
        "or_encode_tensor_v4": (None, [_f32p, _sz, _u8p]),
        "or_encode_tensor_v3": (None, [_f32p, _sz, _u8p]),
        "or_matvec_v4_scalar": (C.c_float, [_u8p, _f32p, _sz]),
        "or_matvec_v4_fused": (C.c_float, [_u8p, _f32p, _sz]),
        "or_matvec_v3_scalar": (C.c_float, [_u8p, _f32p, _sz]),
        "or_matvec_v3_fused": (C.c_float, [_u8p, _f32p, _sz]),
        "or_matvec_v2_scalar": (C.c_float, [_u8p, _f32p, _sz]),
        "or_have_avx2_fma": (C.c_int, []),
        "or_matvec_v4_fused_avx2": (C.c_int, [_u8p, _f32p, _sz, C.POINTER(C.c_float)]),
        "or_matvec_v3_fused_avx2": (C.c_int, [_u8p, _f32p, _sz, C.POINTER(C.c_float)]),
        "or_linear_v4_matvec": (None, [_u8p, _sz, _sz, _f32p, C.c_void_p, _f32p, C.c_int, C.c_int]),
        "or_linear_v3_matvec": (None, [_u8p, _sz, _sz, _f32p, C.c_void_p, _f32p, C.c_int, C.c_int]),
        "or_linear_v4_matmul": (None, [_u8p, _sz, _sz, _f32p, _sz, _f32p, C.c_int, C.c_int]),
        "or_embed_v4": (None, [_u8p, _sz, C.c_uint32, _f32p]),
        "or_embed_v3": (None, [_u8p, _sz, C.c_uint32, _f32p]),
        "or_dense_matvec": (None, [_f32p, _sz, _sz, _f32p, C.c_void_p, _f32p]),
        "or_softmax_inplace": (None, [_f32p, _sz]),
        "or_rms_norm": (None, [_f32p, _f32p, _sz, C.c_float, _f32p]),
        "or_apply_rope": (None, [_f32p, _sz, _sz, C.c_double]),
        "or_argmax": (C.c_uint32, [_f32p, _sz]),
        "or_silu_mul": (C.c_float, [C.c_float, C.c_float]),
        "or_route": (_sz, [_f32p, _sz, _sz, C.c_int, _i32p, _f32p]),
        "or_silu_mul_array": (None, [_f32p, _f32p, _f32p, _sz]),
        "or_kv_cache_new": (C.c_void_p, [C.c_void_p, _sz]),
        "or_kv_cache_free": (None, [C.c_void_p]),
        "or_kv_cache_len": (_sz, [C.c_void_p]),
        "or_forward_token_v4": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, _f32p, C.c_int, C.c_int]),
        "or_moe_ffn_v4": (None, [_f32p, _sz, _sz, _sz, _sz, C.c_int, C.c_void_p, _f32p, _f32p,
                                 _i32p, _f32p, C.c_int, C.c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def _ptr_or_none(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- f16
def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_array(h.ravel(), out.ravel(), h.size)
    return out


def f32_to_f16(f) -> np.ndarray:
    f = _f32(f)
    out = np.empty(f.shape, np.uint16)
    lib().or_f32_to_f16_array(f.ravel(), out.ravel(), f.size)
    return out


# ---------------------------------------------------------------- codecs
def v4_pack(codes) -> np.ndarray:
    codes = _u8(codes)
    out = np.empty(64, np.uint8)
    lib().or_v4_pack_codes(codes, out)
    return out


def v4_unpack(packed) -> np.ndarray:
    out = np.empty(128, np.uint8)
    lib().or_v4_unpack_codes(_u8(packed), out)
    return out


def v3_pack(codes) -> np.ndarray:
    out = np.empty(96, np.uint8)
    lib().or_v3_pack_codes(_u8(codes), out)
    return out


def v3_unpack(packed) -> np.ndarray:
    out = np.empty(128, np.uint8)
    lib().or_v3_unpack_codes(_u8(packed), out)
    return out


def v3tp_pack(codes):
    lp, hp = np.empty(64, np.uint8), np.empty(32, np.uint8)
    lib().or_v3tp_pack(_u8(codes), lp, hp)
    return lp, hp


def v3tp_unpack(lp, hp) -> np.ndarray:
    out = np.empty(128, np.uint8)
    lib().or_v3tp_unpack(_u8(lp), _u8(hp), out)
    return out


# ---------------------------------------------------------------- encoder
def quant_block_v2(w) -> np.ndarray:
    out = np.empty(132, np.uint8)
    lib().or_affine_quant_block_v2(_f32(w), out)
    return out


def quant_block_v3(w) -> np.ndarray:
    out = np.empty(100, np.uint8)
    lib().or_affine_quant_block_v3(_f32(w), out)
    return out


def quant_block_v4(w) -> np.ndarray:
    out = np.empty(68, np.uint8)
    lib().or_affine_quant_block_v4(_f32(w), out)
    return out


def encode_tensor_v4(data) -> np.ndarray:
    data = _f32(data).ravel()
    out = np.empty((data.size // 128) * 68, np.uint8)
    lib().or_encode_tensor_v4(data, data.size, out)
    return out


def encode_tensor_v3(data) -> np.ndarray:
    data = _f32(data).ravel()
    out = np.empty((data.size // 128) * 100, np.uint8)
    lib().or_encode_tensor_v3(data, data.size, out)
    return out


# ---------------------------------------------------------------- kernels
def matvec_row(scheme: int, kernel: int, blocks, x) -> float:
    """One row dot: kernel 0 scalar, 1 fused restatement, 2 AVX2 intrinsics."""
    blocks, x = _u8(blocks), _f32(x)
    bpb = {4: 68, 3: 100, 2: 132}[scheme]
    nb = blocks.size // bpb
    L = lib()
    if kernel == KERNEL_AVX2:
        out = C.c_float()
        fn = L.or_matvec_v4_fused_avx2 if scheme == 4 else L.or_matvec_v3_fused_avx2
        if not fn(blocks, x, nb, C.byref(out)):
            raise RuntimeError("CPU lacks AVX2+FMA")
        return out.value
    fn = {
        (4, 0): L.or_matvec_v4_scalar, (4, 1): L.or_matvec_v4_fused,
        (3, 0): L.or_matvec_v3_scalar, (3, 1): L.or_matvec_v3_fused,
        (2, 0): L.or_matvec_v2_scalar,
    }[(scheme, kernel)]
    return float(fn(blocks, x, nb))


def have_avx2() -> bool:
    return bool(lib().or_have_avx2_fma())


def linear_matvec(scheme: int, blocks, out_f: int, in_f: int, x, bias=None,
                  kernel: int = KERNEL_FUSED, threads: int = 1) -> np.ndarray:
    """WpcLinearV{3,4}::matvec over reference-layout blocks."""
    blocks, x = _u8(blocks), _f32(x)
    y = np.empty(out_f, np.float32)
    b = None if bias is None else _f32(bias)
    fn = lib().or_linear_v4_matvec if scheme == 4 else lib().or_linear_v3_matvec
    fn(blocks, out_f, in_f, x, _ptr_or_none(b), y, kernel, threads)
    return y


def linear_matmul_v4(blocks, out_f, in_f, X, kernel=KERNEL_FUSED, threads=1):
    X = _f32(X)
    M = X.shape[0]
    Y = np.empty((M, out_f), np.float32)
    lib().or_linear_v4_matmul(_u8(blocks), out_f, in_f, X.ravel(), M, Y.ravel(), kernel, threads)
    return Y


def embed(scheme: int, blocks, hidden: int, token: int) -> np.ndarray:
    out = np.empty(hidden, np.float32)
    fn = lib().or_embed_v4 if scheme == 4 else lib().or_embed_v3
    fn(_u8(blocks), hidden, token, out)
    return out


# ---------------------------------------------------------------- dense ops
def dense_matvec(W, x, bias=None) -> np.ndarray:
    W = _f32(W)
    out_f, in_f = W.shape
    y = np.empty(out_f, np.float32)
    b = None if bias is None else _f32(bias)
    lib().or_dense_matvec(W.ravel(), out_f, in_f, _f32(x), _ptr_or_none(b), y)
    return y


def softmax(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().or_softmax_inplace(x, x.size)
    return x


def rms_norm(x, w, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().or_rms_norm(x, w, x.size, eps, out)
    return out


def apply_rope(x, pos: int, theta: float) -> np.ndarray:
    x = _f32(x).copy()
    lib().or_apply_rope(x, x.size, pos, theta)
    return x


def argmax(logits) -> int:
    logits = _f32(logits)
    return int(lib().or_argmax(logits, logits.size))


def silu_mul(g: float, u: float) -> float:
    return float(lib().or_silu_mul(g, u))


def route(scores, top_k: int, norm_topk: bool):
    scores = _f32(scores)
    ids = np.full(max(top_k, 1), -1, np.int32)
    w = np.zeros(max(top_k, 1), np.float32)
    n = lib().or_route(scores, scores.size, top_k, int(norm_topk), ids, w)
    return ids[:n].copy(), w[:n].copy()


def silu_mul_array(g, u) -> np.ndarray:
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    lib().or_silu_mul_array(g, u, out, g.size)
    return out


class _Expert(C.Structure):
    _fields_ = [("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p)]


def moe_ffn_v4(router_w, experts, x, top_k: int, norm_topk: bool = True,
               kernel: int = KERNEL_FUSED, threads: int = 4):
    """or_moe_ffn_v4: (mlp_out, ids, weights). experts: [(gate, up, down)]
    reference v4 blocks per expert; router_w [n_exp, hidden] fp32."""
    router_w = np.ascontiguousarray(router_w, np.float32)
    n_exp, hidden = router_w.shape
    x = _f32(x)
    keep = [tuple(np.ascontiguousarray(b, np.uint8) for b in e) for e in experts]
    inter = keep[0][0].size // 68 // (hidden // 128)
    arr = (_Expert * n_exp)(*[_Expert(g.ctypes.data, u.ctypes.data, d.ctypes.data) for g, u, d in keep])
    out = np.empty(hidden, np.float32)
    ids = np.empty(top_k, np.int32)
    w = np.empty(top_k, np.float32)
    lib().or_moe_ffn_v4(router_w.ravel(), n_exp, hidden, inter, top_k, int(bool(norm_topk)),
                        C.cast(arr, C.c_void_p), x, out, ids, w, kernel, threads)
    return out, ids, w



class _Cfg(C.Structure):
    _fields_ = [(f, C.c_size_t) for f in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim",
                                          "inter", "vocab", "n_exp", "top_k", "moe_inter")] + [
        ("norm_topk", C.c_int), ("rope_theta", C.c_double), ("eps", C.c_float)]


class _Layer(C.Structure):
    _fields_ = [(f, C.c_void_p) for f in ("input_ln", "post_ln", "q_norm", "k_norm", "q", "k", "v", "o",
                                          "gate", "up", "down", "router", "experts")]


class _Model(C.Structure):
    _fields_ = [("cfg", _Cfg), ("embed", C.c_void_p), ("lm_head", C.c_void_p),
                ("final_norm", C.c_void_p), ("layers", C.c_void_p)]


class Model:
    """or_forward_token_v4: the reference's dense Qwen3 / Qwen3-MoE decode
    step on the CPU (v4 weights). cfg: dict with the wpcg.ModelConfig field
    names; tensors: {reference name: array}."""

    def __init__(self, cfg: dict, tensors: dict, max_pos: int, kernel: int = KERNEL_FUSED,
                 threads: int = 8):
        self.cfg, self.kernel, self.threads = cfg, kernel, threads
        self.keep = {k: np.ascontiguousarray(v) for k, v in tensors.items()}
        T = self.keep
        ptr = lambda n: T[n].ctypes.data if n in T else None  # noqa: E731
        L = cfg["n_layers"]
        self.layers = (_Layer * L)()
        self.expert_arrays = []
        for l in range(L):
            p = f"model.layers.{l}."
            lay = self.layers[l]
            lay.input_ln, lay.post_ln = ptr(p + "input_layernorm.weight"), ptr(p + "post_attention_layernorm.weight")
            lay.q_norm, lay.k_norm = ptr(p + "self_attn.q_norm.weight"), ptr(p + "self_attn.k_norm.weight")
            lay.q, lay.k = ptr(p + "self_attn.q_proj.weight"), ptr(p + "self_attn.k_proj.weight")
            lay.v, lay.o = ptr(p + "self_attn.v_proj.weight"), ptr(p + "self_attn.o_proj.weight")
            if cfg["n_experts"]:
                E = cfg["n_experts"]
                arr = (_Expert * E)(*[_Expert(ptr(p + f"mlp.experts.{e}.gate_proj.weight"),
                                              ptr(p + f"mlp.experts.{e}.up_proj.weight"),
                                              ptr(p + f"mlp.experts.{e}.down_proj.weight")) for e in range(E)])
                self.expert_arrays.append(arr)
                lay.router, lay.experts = ptr(p + "mlp.gate.weight"), C.cast(arr, C.c_void_p)
            else:
                lay.gate, lay.up = ptr(p + "mlp.gate_proj.weight"), ptr(p + "mlp.up_proj.weight")
                lay.down = ptr(p + "mlp.down_proj.weight")
        c = _Cfg(cfg["n_layers"], cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"],
                 cfg["inter"], cfg["vocab"], cfg["n_experts"], cfg["top_k"], cfg["moe_inter"],
                 int(cfg["norm_topk"]), float(cfg["rope_theta"]), float(cfg["eps"]))
        self.model = _Model(c, ptr("model.embed_tokens.weight"), ptr("lm_head.weight"),
                            ptr("model.norm.weight"), C.cast(self.layers, C.c_void_p))
        self.cache = lib().or_kv_cache_new(C.byref(self.model.cfg), max_pos)

    def forward_token(self, token: int, threads: int | None = None) -> np.ndarray:
        """One step; `threads` overrides the model's thread count for this call."""
        logits = np.empty(self.cfg["vocab"], np.float32)
        rc = lib().or_forward_token_v4(C.byref(self.model), token, self.cache, logits, self.kernel,
                                       self.threads if threads is None else threads)
        assert rc == 0, rc
        return logits

    def close(self):
        if self.cache:
            lib().or_kv_cache_free(self.cache)
            self.cache = None

    def __del__(self):
        self.close()
