"""ORACLE -- test infrastructure only. ctypes access to the two CPU implementations
of glm.c's MoE path behind oracle/oracle.h:

  Oracle("port")       oracle/liboracle.so, the C restatement (moe_oracle.c)
  Oracle("reference")  oracle/_ref/libref_moe.so, glm.c's own infer.c compiled by oracle/Makefile

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import this.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PATHS = {"port": os.path.join(HERE, "liboracle.so"), "reference": os.path.join(HERE, "_ref", "libref_moe.so")}
PREFIX = {"port": "oracle_", "reference": "ref_"}


class Dims(C.Structure):
    _fields_ = [("dim", C.c_int32), ("moe_ffn_dim", C.c_int32), ("n_routed_experts", C.c_int32),
                ("n_experts_used", C.c_int32), ("group_size", C.c_int32)]


_LAYER_FIELDS = ["ffn_norm", "gate_inp", "exp_probs_b", "gate_sh_q", "gate_sh_s", "up_sh_q", "up_sh_s",
                 "down_sh_q", "down_sh_s", "gate_q", "gate_s", "up_q", "up_s", "down_q", "down_s"]


class Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _LAYER_FIELDS]


class Out(C.Structure):
    _fields_ = [("x_out", C.c_void_p), ("xn", C.c_void_p), ("router_prob", C.c_void_p), ("topk_idx", C.c_void_p),
                ("topk_w", C.c_void_p), ("shared_out", C.c_void_p), ("routed_out", C.c_void_p)]


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def available(kind):
    return os.path.exists(PATHS[kind])


def layer_struct(host_layer):
    return Layer(*[_p(getattr(host_layer, n)) for n in _LAYER_FIELDS])


class Oracle:
    def __init__(self, kind="port"):
        if not available(kind):
            raise RuntimeError(f"oracle '{kind}' not built: {PATHS[kind]}")
        self.kind = kind
        self.lib = C.CDLL(PATHS[kind])
        pre = PREFIX[kind]
        self._layer = getattr(self.lib, pre + "moe_layer")
        self._layer.argtypes = [C.POINTER(Dims), C.POINTER(Layer), C.c_int, C.c_void_p, C.POINTER(Out), C.c_int]
        self._layer.restype = C.c_int
        self._stack = getattr(self.lib, pre + "moe_stack")
        self._stack.argtypes = [C.POINTER(Dims), C.POINTER(Layer), C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        self._stack.restype = C.c_int
        if kind == "reference":
            L = self.lib
            L.ref_moe_stack_timed.argtypes = [C.POINTER(Dims), C.POINTER(Layer), C.c_int, C.c_int, C.c_void_p,
                                              C.c_void_p, C.c_int]
            L.ref_moe_stack_timed.restype = C.c_int
            L.ref_moe_layer_timed.argtypes = [C.POINTER(Dims), C.POINTER(Layer), C.c_int, C.c_void_p, C.c_void_p,
                                              C.c_int]
            L.ref_moe_layer_timed.restype = C.c_int
        if kind == "port":
            L = self.lib
            L.oracle_dispatch.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
            L.oracle_dispatch.restype = C.c_int
            L.oracle_rmsnorm.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
            L.oracle_router_logits.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]
            L.oracle_sigmoid.argtypes = [C.c_float]
            L.oracle_sigmoid.restype = C.c_float
            L.oracle_silu.argtypes = [C.c_float]
            L.oracle_silu.restype = C.c_float
            L.oracle_topk.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
            L.oracle_matvec_q8.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]
            L.oracle_expf_compare.argtypes = [C.c_uint32, C.c_int64, C.c_void_p, C.c_int, C.POINTER(C.c_int64)]
            L.oracle_expf_compare.restype = C.c_int64

    @staticmethod
    def dims(shape):
        return Dims(shape.D, shape.F, shape.E, shape.K, shape.gs)

    def layer(self, shape, host_layer, x, disable_routed=False):
        """Run T tokens through one layer; returns a dict of the observable outputs."""
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        D, E, K = shape.D, shape.E, shape.K
        res = {"x_out": np.zeros((T, D), np.float32), "xn": np.zeros((T, D), np.float32),
               "router_prob": np.zeros((T, E), np.float32), "topk_idx": np.zeros((T, K), np.int32),
               "topk_w": np.zeros((T, K), np.float32), "shared_out": np.zeros((T, D), np.float32),
               "routed_out": np.zeros((T, D), np.float32)}
        out = Out(*[_p(res[n]) for n, _ in Out._fields_])
        rc = self._layer(C.byref(self.dims(shape)), C.byref(layer_struct(host_layer)), T, _p(x), C.byref(out),
                         1 if disable_routed else 0)
        if rc != 0:
            raise RuntimeError("oracle layer failed")
        return res

    def stack(self, shape, host_layers, x):
        """Run T tokens through the layers in sequence; returns (x_out, topk_idx[L][T][K])."""
        x = np.array(x, np.float32, copy=True)
        T = x.shape[0]
        arr = (Layer * len(host_layers))(*[layer_struct(h) for h in host_layers])
        topk = np.zeros((len(host_layers), T, shape.K), np.int32)
        rc = self._stack(C.byref(self.dims(shape)), arr, len(host_layers), T, _p(x), _p(topk))
        if rc != 0:
            raise RuntimeError("oracle stack failed")
        return x, topk


def stack_timed(shape, host_layers, x, n_tokens, n_threads=0):
    """CPU baseline: n_tokens decode tokens through the reference build's stack from x;
    returns the per-layer-call wall times in ms, [n_tokens][n_layers]."""
    orc = Oracle("reference")
    x = np.array(x, np.float32, copy=True).reshape(-1)
    arr = (Layer * len(host_layers))(*[layer_struct(h) for h in host_layers])
    ms = np.zeros((n_tokens, len(host_layers)), np.float64)
    rc = orc.lib.ref_moe_stack_timed(C.byref(Oracle.dims(shape)), arr, len(host_layers), n_tokens, _p(x), _p(ms),
                                     n_threads)
    if rc != 0:
        raise RuntimeError("ref_moe_stack_timed failed")
    return ms


def layer_timed(shape, host_layer, x, n_threads=0):
    """CPU baseline: every token of x through one layer of the reference build, one timed
    call each; returns the per-token wall times in ms."""
    orc = Oracle("reference")
    x = np.ascontiguousarray(x, np.float32)
    ms = np.zeros(x.shape[0], np.float64)
    rc = orc.lib.ref_moe_layer_timed(C.byref(Oracle.dims(shape)), C.byref(layer_struct(host_layer)), x.shape[0],
                                     _p(x), _p(ms), n_threads)
    if rc != 0:
        raise RuntimeError("ref_moe_layer_timed failed")
    return ms


def expf_compare(first_bits, got, max_ulp=0):
    """(mismatches, first mismatching bit pattern or -1) of `got` against libm's expf on
    the fp32 inputs with bit patterns first_bits, first_bits + 1, ..."""
    lib = Oracle("port").lib
    got = np.ascontiguousarray(got, np.float32)
    where = C.c_int64(-1)
    n = lib.oracle_expf_compare(first_bits, got.size, _p(got), max_ulp, C.byref(where))
    return int(n), int(where.value)


def dispatch(topk_idx, n_experts):
    """Per-expert token lists from [T][K] top-k indices (oracle_dispatch)."""
    lib = Oracle("port").lib
    t = np.ascontiguousarray(topk_idx, np.int32)
    T, K = t.shape
    offsets = np.zeros(n_experts + 1, np.int32)
    tokens = np.zeros(max(1, T * K), np.int32)
    slots = np.zeros(max(1, T * K), np.int32)
    n = lib.oracle_dispatch(T, K, n_experts, _p(t), _p(offsets), _p(tokens), _p(slots))
    if n < 0:
        raise RuntimeError("oracle_dispatch failed")
    return offsets, tokens[:n], slots[:n]
