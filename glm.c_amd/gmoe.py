"""ctypes bindings for the MI355X MoE FFN path.

libgmoe.so      kernels behind the C ABI of include/gmoe.h
libglm_hip.so   C host side: glm.c's backend interface with BACKEND_HIP
                (include/glm_backend.h) and the synthetic-input generator

This module is plumbing for tests and the benchmark: it allocates host arrays
in glm.c's checkpoint layout (model.h:65-84) and hands raw pointers to the C
ABI. It never computes a result itself, and it raises if the native libraries
are missing: there is no fallback path.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIBGMOE = os.environ.get("GMOE_LIBRARY", os.path.join(HERE, "libgmoe.so"))
LIBHOST = os.path.join(HERE, "libglm_hip.so")

GMOE_FLAG_NO_ROUTED = 1
GMOE_FLAG_EXACT_ROUTER = 2
# gmoe_config.q8_form: device form of the expert matrices
GMOE_Q8_AUTO, GMOE_Q8_TILED, GMOE_Q8_NATIVE, GMOE_Q8_TILED16 = 0, 1, 2, 3
SYNTH_NORM_ONES, SYNTH_NORM_RANDOM = 0, 1
SYNTH_BIAS_NORMAL, SYNTH_BIAS_ZIPF = 0, 1
SYNTH_SCALES_FP16, SYNTH_SCALES_FP32 = 0, 1

# Zipf-shaped router bias for the skewed-routing workload: popularity ~ rank^-1.2,
# gain chosen so the 4 most popular experts take about 40% of top-4 assignments.
ZIPF_S = 1.2
ZIPF_BETA = 0.095


class GmoeConfig(C.Structure):
    _fields_ = [("dim", C.c_int32), ("moe_ffn_dim", C.c_int32), ("n_routed_experts", C.c_int32),
                ("n_experts_used", C.c_int32), ("n_shared_experts", C.c_int32), ("group_size", C.c_int32),
                ("n_layers", C.c_int32), ("max_tokens", C.c_int32), ("routed_scale", C.c_float),
                ("norm_eps", C.c_float), ("q8_form", C.c_int32)]


_LAYER_FIELDS = ["ffn_norm", "gate_inp", "exp_probs_b", "gate_sh_q", "gate_sh_s", "up_sh_q", "up_sh_s",
                 "down_sh_q", "down_sh_s", "gate_q", "gate_s", "up_q", "up_s", "down_q", "down_s"]


class LayerWeights(C.Structure):
    """gmoe_layer_weights / oracle_layer / synth_layer_buffers: 15 pointers, same order."""
    _fields_ = [(n, C.c_void_p) for n in _LAYER_FIELDS]


class GmoeLayerState(C.Structure):
    _fields_ = [("xn", C.c_void_p), ("router_prob", C.c_void_p), ("topk_idx", C.c_void_p), ("topk_w", C.c_void_p),
                ("shared_out", C.c_void_p), ("routed_out", C.c_void_p), ("expert_offsets", C.c_void_p),
                ("expert_tokens", C.c_void_p)]


# gmoe_profile buckets (GMOE_KERNEL_*): gate_up is k_gate_up (T=1) or k_group_gu (grouped
# prefill), down is k_down_combine or k_group_down
KERNEL_NAMES = {0: "k_router_tok", 1: "gate_up", 2: "down", 3: "k_dispatch", 4: "k_moe_stack", 5: "k_act_split",
                6: "k_token_combine", 8: "k_moe_relay"}
N_KERNEL_IDS = 9


class GmoeKernelTimes(C.Structure):
    _fields_ = [("launches", C.c_int64 * N_KERNEL_IDS), ("ms", C.c_double * N_KERNEL_IDS)]


class GmoeStats(C.Structure):
    _fields_ = [("tokens_routed", C.c_int64), ("routing_exact_path", C.c_int64), ("routing_exact_subset", C.c_int64),
                ("norm_exact_path", C.c_int64),
                ("scale_inexact", C.c_int64), ("expf_libc_match", C.c_int64), ("q8_form", C.c_int64)]


class SynthSpec(C.Structure):
    _fields_ = [("seed", C.c_uint64), ("dim", C.c_int32), ("moe_ffn_dim", C.c_int32),
                ("n_routed_experts", C.c_int32), ("group_size", C.c_int32), ("norm_mode", C.c_int32),
                ("bias_mode", C.c_int32), ("zipf_s", C.c_double), ("zipf_beta", C.c_double),
                ("scale_mode", C.c_int32)]


_libs = {}


def _load(path, what):
    if path in _libs:
        return _libs[path]
    if not os.path.exists(path):
        raise RuntimeError(f"{what} not built: {path} is missing (run __graft_entry__.build())")
    lib = C.CDLL(path, mode=C.RTLD_GLOBAL)
    _libs[path] = lib
    return lib


def host_lib():
    lib = _load(LIBHOST, "host library")
    if not getattr(lib, "_typed", False):
        lib.synth_layer.argtypes = [C.POINTER(SynthSpec), C.c_int, C.c_int, C.c_int, C.POINTER(LayerWeights)]
        lib.synth_layer.restype = C.c_int
        lib.synth_activations.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_void_p]
        lib.synth_activations.restype = None
        lib.synth_round_fp16.argtypes = [C.c_float]
        lib.synth_round_fp16.restype = C.c_float
        lib.synth_key.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int]
        lib.synth_key.restype = C.c_uint64
        lib.synth_draw.argtypes = [C.c_uint64, C.c_uint64]
        lib.synth_draw.restype = C.c_uint64
        lib.synth_q8_at.argtypes = [C.c_uint64, C.c_uint64]
        lib.synth_q8_at.restype = C.c_int
        lib.synth_normal_at.argtypes = [C.c_uint64, C.c_uint64]
        lib.synth_normal_at.restype = C.c_double
        lib.synth_q8_matrix.argtypes = [C.c_uint64, C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                        C.c_void_p]
        lib.synth_q8_matrix.restype = None
        lib.synth_normal_fill.argtypes = [C.c_uint64, C.c_size_t, C.c_double, C.c_double, C.c_void_p]
        lib.synth_normal_fill.restype = None
        lib._typed = True
    return lib


def gmoe_lib():
    lib = _load(LIBGMOE, "HIP library")
    if not getattr(lib, "_typed", False):
        P = C.c_void_p
        lib.gmoe_create.argtypes = [C.POINTER(P), C.c_int, C.POINTER(GmoeConfig)]
        lib.gmoe_upload_layer.argtypes = [P, C.c_int, C.POINTER(LayerWeights)]
        lib.gmoe_forward.argtypes = [P, C.c_int, C.c_int, P, P, C.c_int, P]
        lib.gmoe_forward_layers.argtypes = [P, C.c_int, C.c_int, C.c_int, P, P, C.c_int, P]
        lib.gmoe_read_layer_state.argtypes = [P, C.POINTER(GmoeLayerState), P]
        lib.gmoe_read_topk.argtypes = [P, C.c_int, P, P, P]
        lib.gmoe_get_stats.argtypes = [P, C.POINTER(GmoeStats)]
        lib.gmoe_expert_bytes_last.argtypes = [P]
        lib.gmoe_expert_bytes_last.restype = C.c_int64
        lib.gmoe_profile.argtypes = [P, C.c_int]
        lib.gmoe_profile.restype = C.c_int
        lib.gmoe_profile_read.argtypes = [P, C.POINTER(GmoeKernelTimes)]
        lib.gmoe_profile_read.restype = C.c_int
        lib.gmoe_forward_host.argtypes = [P, C.c_int, C.c_int, P, P, C.c_int, P]
        lib.gmoe_forward_host.restype = C.c_int
        lib.gmoe_expf_eval.argtypes = [C.c_uint32, C.c_int64, C.c_int, P, P]
        lib.gmoe_expf_eval.restype = C.c_int
        lib.gmoe_destroy.argtypes = [P]
        lib.gmoe_destroy.restype = None
        lib.gmoe_last_error.argtypes = []
        lib.gmoe_last_error.restype = C.c_char_p
        for f in ("gmoe_create", "gmoe_upload_layer", "gmoe_forward", "gmoe_forward_layers",
                  "gmoe_read_layer_state", "gmoe_read_topk", "gmoe_get_stats"):
            getattr(lib, f).restype = C.c_int
        lib._typed = True
    return lib


def ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Shape:
    """MoE layer shape (RuntimeConfig fields, model.h:7-45)."""

    def __init__(self, dim=2048, moe_ffn_dim=1536, n_routed_experts=64, n_experts_used=4, group_size=32):
        self.D, self.F, self.E, self.K, self.gs = dim, moe_ffn_dim, n_routed_experts, n_experts_used, group_size

    def expert_bytes(self):
        """Algorithmic Q8_0 bytes of one expert as the device keeps it: three matrices of int8
        weights plus one scale per group, fp16 at group size 32 (34 bytes per 32 weights), fp32
        otherwise (20 bytes per 16 weights at the exporter's group size 16)."""
        sb = 2 if self.gs == 32 else 4
        return 3 * self.F * self.D * (self.gs + sb) // self.gs


GLM47_FLASH = Shape()


class HostLayer:
    """One MoE layer's weights in glm.c's checkpoint layout, as numpy arrays.

    Arrays come from np.zeros, so routed experts that are never generated cost
    no resident memory."""

    def __init__(self, shape, seed=0, layer=1, experts=None, norm_mode=SYNTH_NORM_ONES,
                 bias_mode=SYNTH_BIAS_NORMAL, zipf_s=ZIPF_S, zipf_beta=ZIPF_BETA, routed=True,
                 scale_mode=SYNTH_SCALES_FP16):
        s = shape
        self.shape, self.seed, self.layer = s, seed, layer
        D, F, E, gs = s.D, s.F, s.E, s.gs
        self.ffn_norm = np.zeros(D, np.float32)
        self.gate_inp = np.zeros((E, D), np.float32)
        self.exp_probs_b = np.zeros(E, np.float32)
        self.gate_sh_q = np.zeros((F, D), np.int8)
        self.gate_sh_s = np.zeros((F, D // gs), np.float32)
        self.up_sh_q = np.zeros((F, D), np.int8)
        self.up_sh_s = np.zeros((F, D // gs), np.float32)
        self.down_sh_q = np.zeros((D, F), np.int8)
        self.down_sh_s = np.zeros((D, F // gs), np.float32)
        if routed:
            self.gate_q = np.zeros((E, F, D), np.int8)
            self.gate_s = np.zeros((E, F, D // gs), np.float32)
            self.up_q = np.zeros((E, F, D), np.int8)
            self.up_s = np.zeros((E, F, D // gs), np.float32)
            self.down_q = np.zeros((E, D, F), np.int8)
            self.down_s = np.zeros((E, D, F // gs), np.float32)
        else:
            self.gate_q = self.gate_s = self.up_q = self.up_s = self.down_q = self.down_s = None
        spec = SynthSpec(seed, D, F, E, gs, norm_mode, bias_mode, zipf_s, zipf_beta, scale_mode)
        e0, e1 = (0, E) if experts is None else experts
        if not routed:
            e0 = e1 = 0
        rc = host_lib().synth_layer(C.byref(spec), layer, e0, e1, C.byref(self.weights()))
        if rc != 0:
            raise RuntimeError("synth_layer failed")

    def weights(self):
        return LayerWeights(*[ptr(getattr(self, n)) for n in _LAYER_FIELDS])


def activations(seed, stream, n_tokens, dim):
    x = np.empty((n_tokens, dim), np.float32)
    host_lib().synth_activations(seed, stream, n_tokens, dim, ptr(x))
    return x


def last_error():
    e = gmoe_lib().gmoe_last_error()
    return e.decode() if e else ""


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")


class Context:
    """A gmoe_ctx: weights resident on one device, forward calls on device pointers."""

    def __init__(self, shape, n_layers, max_tokens, device=0, routed_scale=1.8, norm_eps=1e-5, n_shared=1,
                 q8_form=GMOE_Q8_AUTO):
        self.lib = gmoe_lib()
        self.shape = shape
        self.max_tokens = max_tokens
        cfg = GmoeConfig(shape.D, shape.F, shape.E, shape.K, n_shared, shape.gs, n_layers, max_tokens,
                         routed_scale, norm_eps, q8_form)
        h = C.c_void_p()
        check(self.lib.gmoe_create(C.byref(h), device, C.byref(cfg)), "gmoe_create")
        self.h = h

    def upload(self, layer, host_layer):
        check(self.lib.gmoe_upload_layer(self.h, layer, C.byref(host_layer.weights())), "gmoe_upload_layer")

    def forward(self, layer, n_tokens, x_in_dev, x_out_dev, flags=0, stream=None):
        check(self.lib.gmoe_forward(self.h, layer, n_tokens, x_in_dev, x_out_dev, flags, stream), "gmoe_forward")

    def forward_layers(self, first, n_layers, n_tokens, x_in_dev, x_out_dev, flags=0, stream=None):
        check(self.lib.gmoe_forward_layers(self.h, first, n_layers, n_tokens, x_in_dev, x_out_dev, flags, stream),
              "gmoe_forward_layers")

    def read_state(self, n_tokens, stream=None):
        s = self.shape
        out = {
            "xn": np.zeros((n_tokens, s.D), np.float32),
            "router_prob": np.zeros((n_tokens, s.E), np.float32),
            "topk_idx": np.zeros((n_tokens, s.K), np.int32),
            "topk_w": np.zeros((n_tokens, s.K), np.float32),
            "shared_out": np.zeros((n_tokens, s.D), np.float32),
            "routed_out": np.zeros((n_tokens, s.D), np.float32),
            "expert_offsets": np.zeros(s.E + 1, np.int32),
            "expert_tokens": np.zeros(max(1, n_tokens * s.K), np.int32),
        }
        st = GmoeLayerState(*[ptr(out[n]) for n, _ in GmoeLayerState._fields_])
        check(self.lib.gmoe_read_layer_state(self.h, C.byref(st), stream), "gmoe_read_layer_state")
        return out

    def read_topk(self, layer, n_tokens, stream=None):
        idx = np.zeros((n_tokens, self.shape.K), np.int32)
        w = np.zeros((n_tokens, self.shape.K), np.float32)
        check(self.lib.gmoe_read_topk(self.h, layer, ptr(idx), ptr(w), stream), "gmoe_read_topk")
        return idx, w

    def stats(self):
        st = GmoeStats()
        check(self.lib.gmoe_get_stats(self.h, C.byref(st)), "gmoe_get_stats")
        return {n: getattr(st, n) for n, _ in GmoeStats._fields_}

    def profile(self, enable):
        check(self.lib.gmoe_profile(self.h, 1 if enable else 0), "gmoe_profile")

    def profile_read(self):
        """{kernel name: (launches, total ms)} from the HIP events of the profiled calls."""
        kt = GmoeKernelTimes()
        check(self.lib.gmoe_profile_read(self.h, C.byref(kt)), "gmoe_profile_read")
        return {KERNEL_NAMES.get(i, str(i)): (int(kt.launches[i]), float(kt.ms[i])) for i in range(N_KERNEL_IDS)
                if kt.launches[i] > 0}

    def expert_bytes_last(self):
        return int(self.lib.gmoe_expert_bytes_last(self.h))

    def close(self):
        if self.h:
            self.lib.gmoe_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------- the whole model (gmoe_model.h)
_MODEL_CFG = ["dim", "hidden_dim", "n_layers", "n_heads", "vocab_size", "q_lora_rank", "kv_lora_rank", "rope_dim",
              "qk_nope_dim", "head_k_dim", "v_head_dim", "group_size", "cache_cap", "attn_layers", "has_l0_ffn",
              "max_batch"]
_ATTN_FIELDS = ["attn_norm", "q_a_norm", "kv_a_norm", "q_a_q", "q_a_s", "q_b_q", "q_b_s", "kv_a_q", "kv_a_s", "k_b_q",
                "k_b_s", "v_b_q", "v_b_s", "attn_out_q", "attn_out_s"]
_MODEL_FIELDS = ["output_norm", "tok_q", "tok_s", "out_q", "out_s", "l0_ffn_norm", "l0_ffn_gate_q", "l0_ffn_gate_s",
                 "l0_ffn_up_q", "l0_ffn_up_s", "l0_ffn_down_q", "l0_ffn_down_s"]


class ModelConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in _MODEL_CFG]


class AttnWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _ATTN_FIELDS]


class ModelWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _MODEL_FIELDS]


# GLM-4.7-Flash's dense side (47 layers, MLA attention on every layer, dense layer 0)
GLM47_FLASH_MODEL = dict(dim=2048, hidden_dim=10240, n_layers=47, n_heads=20, vocab_size=154880, q_lora_rank=768,
                         kv_lora_rank=512, rope_dim=64, qk_nope_dim=192, head_k_dim=256, v_head_dim=256, group_size=32)


def synth_model_weights(cfg, seed):
    """Seeded random-init weights for gmoe_model_upload ({name: array}) and for every
    attention layer's gmoe_model_upload_attn ([{name: array}]), from the counter-based
    generator of the MoE layers (synth.c): Q8_0 values uniform in [-127, 127], fp32 scales
    |N(0,1)| * 0.002, norm weights N(1, 0.1). Tensor t of layer l draws from
    synth_key(seed, l, 100 + t, 0) (model-wide tensors: layer -1), apart from every MoE stream."""
    h = host_lib()
    D, gs, H = cfg["dim"], cfg["group_size"], cfg["n_heads"]
    kv, rope, nope, hk, vh = cfg["kv_lora_rank"], cfg["rope_dim"], cfg["qk_nope_dim"], cfg["head_k_dim"], cfg["v_head_dim"]
    where = {"layer": -1, "t": 100}

    def key():
        where["t"] += 1
        return h.synth_key(seed, where["layer"], where["t"], 0)

    def norm(n):
        out = np.empty(n, np.float32)
        h.synth_normal_fill(key(), n, 1.0, 0.1, ptr(out))
        return out

    def q8(rows, cols):
        q = np.empty((rows, cols), np.int8)
        s = np.empty((rows, cols // gs), np.float32)
        h.synth_q8_matrix(key(), key(), rows, cols, gs, SYNTH_SCALES_FP32, ptr(q), ptr(s))
        return q, s

    g = {"output_norm": norm(D)}
    g["tok_q"], g["tok_s"] = q8(cfg["vocab_size"], D)
    g["out_q"], g["out_s"] = q8(cfg["vocab_size"], D)
    if cfg.get("has_l0_ffn", 1):
        F = cfg["hidden_dim"]
        g["l0_ffn_norm"] = norm(D)
        g["l0_ffn_gate_q"], g["l0_ffn_gate_s"] = q8(F, D)
        g["l0_ffn_up_q"], g["l0_ffn_up_s"] = q8(F, D)
        g["l0_ffn_down_q"], g["l0_ffn_down_s"] = q8(D, F)
    layers = []
    for layer in range(cfg.get("attn_layers", cfg["n_layers"])):
        where["layer"], where["t"] = layer, 100
        a = {"attn_norm": norm(D), "q_a_norm": norm(cfg["q_lora_rank"]), "kv_a_norm": norm(kv)}
        a["q_a_q"], a["q_a_s"] = q8(cfg["q_lora_rank"], D)
        a["q_b_q"], a["q_b_s"] = q8(H * hk, cfg["q_lora_rank"])
        a["kv_a_q"], a["kv_a_s"] = q8(kv + rope, D)
        a["k_b_q"], a["k_b_s"] = q8(H * kv, nope)
        a["v_b_q"], a["v_b_s"] = q8(H * vh, kv)
        a["attn_out_q"], a["attn_out_s"] = q8(D, H * vh)
        layers.append(a)
    return g, layers


class Model:
    """A gmoe_model: the whole decode forward on one device (embedding, MLA attention over
    a device-resident latent cache, dense layer 0, the MoE layers of a Context, LM head)."""

    def __init__(self, cfg, device=0):
        self.lib = gmoe_lib()
        if not getattr(self.lib, "_model_typed", False):
            P = C.c_void_p
            self.lib.gmoe_model_create.argtypes = [C.POINTER(P), C.c_int, C.POINTER(ModelConfig)]
            self.lib.gmoe_model_upload.argtypes = [P, C.POINTER(ModelWeights)]
            self.lib.gmoe_model_upload_attn.argtypes = [P, C.c_int, C.POINTER(AttnWeights)]
            self.lib.gmoe_model_set_moe.argtypes = [P, P, P, C.c_int]
            self.lib.gmoe_model_forward_token.argtypes = [P, C.c_int, C.c_int, C.c_int, P, P, P, P, P]
            self.lib.gmoe_model_prefill.argtypes = [P, P, C.c_int, C.c_int, P, P, P]
            for f in ("gmoe_model_create", "gmoe_model_upload", "gmoe_model_upload_attn", "gmoe_model_set_moe",
                      "gmoe_model_forward_token", "gmoe_model_prefill"):
                getattr(self.lib, f).restype = C.c_int
            self.lib.gmoe_model_destroy.argtypes = [P]
            self.lib.gmoe_model_destroy.restype = None
            self.lib._model_typed = True
        self.cfg = dict(cfg)
        mc = ModelConfig(*[int(self.cfg.get(n, 0)) for n in _MODEL_CFG])
        h = C.c_void_p()
        check(self.lib.gmoe_model_create(C.byref(h), device, C.byref(mc)), "gmoe_model_create")
        self.h = h
        self.logits = np.zeros(self.cfg["vocab_size"], np.float32)

    def upload(self, weights):
        w = ModelWeights(*[ptr(weights.get(n)) for n in _MODEL_FIELDS])
        check(self.lib.gmoe_model_upload(self.h, C.byref(w)), "gmoe_model_upload")

    def upload_attn(self, layer, weights):
        w = AttnWeights(*[ptr(weights[n]) for n in _ATTN_FIELDS])
        check(self.lib.gmoe_model_upload_attn(self.h, layer, C.byref(w)), "gmoe_model_upload_attn")

    def set_moe(self, ctx, layers, flags=0):
        on = np.zeros(self.cfg["n_layers"], np.uint8)
        on[list(layers)] = 1
        check(self.lib.gmoe_model_set_moe(self.h, ctx.h, ptr(on), flags), "gmoe_model_set_moe")

    def forward_token(self, token, pos, flags=0, stream=None):
        check(self.lib.gmoe_model_forward_token(self.h, int(token), int(pos), flags, ptr(self.logits), None, None, None,
                                                stream), "gmoe_model_forward_token")
        return self.logits

    def prefill(self, tokens, pos0=0, stream=None):
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        check(self.lib.gmoe_model_prefill(self.h, ptr(toks), int(toks.size), int(pos0), ptr(self.logits), None, stream),
              "gmoe_model_prefill")
        return self.logits

    def close(self):
        if self.h:
            self.lib.gmoe_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------- HIP runtime (ctypes)
_hip = None
HIP_H2D, HIP_D2H, HIP_D2D = 1, 2, 3


def hip():
    """libamdhip64 with the few entry points the tests and the benchmark need."""
    global _hip
    if _hip is not None:
        return _hip
    lib = C.CDLL("libamdhip64.so", mode=C.RTLD_GLOBAL)
    P = C.c_void_p
    sig = {
        "hipGetDeviceCount": [C.POINTER(C.c_int)],
        "hipSetDevice": [C.c_int],
        "hipMalloc": [C.POINTER(P), C.c_size_t],
        "hipFree": [P],
        "hipMemcpy": [P, P, C.c_size_t, C.c_int],
        "hipMemset": [P, C.c_int, C.c_size_t],
        "hipDeviceSynchronize": [],
        "hipStreamCreate": [C.POINTER(P)],
        "hipStreamDestroy": [P],
        "hipStreamSynchronize": [P],
        "hipEventCreate": [C.POINTER(P)],
        "hipEventDestroy": [P],
        "hipEventRecord": [P, P],
        "hipEventSynchronize": [P],
        "hipEventElapsedTime": [C.POINTER(C.c_float), P, P],
        "hipStreamBeginCapture": [P, C.c_int],
        "hipStreamEndCapture": [P, C.POINTER(P)],
        "hipGraphInstantiate": [C.POINTER(P), P, P, P, C.c_size_t],
        "hipGraphLaunch": [P, P],
        "hipGraphExecDestroy": [P],
        "hipGraphDestroy": [P],
    }
    for name, args in sig.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = C.c_int
    lib.hipGetErrorString.argtypes = [C.c_int]
    lib.hipGetErrorString.restype = C.c_char_p
    _hip = lib
    return lib


def hip_check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed: {hip().hipGetErrorString(rc).decode()}")


def device_count():
    n = C.c_int(0)
    rc = hip().hipGetDeviceCount(C.byref(n))
    return n.value if rc == 0 else 0


class DeviceArray:
    """A hipMalloc'd buffer with numpy copy in/out."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        hip_check(hip().hipMalloc(C.byref(p), max(1, self.nbytes)), "hipMalloc")
        self.ptr = p

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        d.upload(a)
        return d

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        hip_check(hip().hipMemcpy(self.ptr, a.ctypes.data_as(C.c_void_p), a.nbytes, HIP_H2D), "hipMemcpy H2D")

    def download(self, shape, dtype):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        hip_check(hip().hipMemcpy(out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes, HIP_D2H), "hipMemcpy D2H")
        return out

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = C.c_void_p()
        hip_check(hip().hipStreamCreate(C.byref(s)), "hipStreamCreate")
        self.h = s

    def sync(self):
        hip_check(hip().hipStreamSynchronize(self.h), "hipStreamSynchronize")


class Event:
    def __init__(self):
        e = C.c_void_p()
        hip_check(hip().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.h = e

    def record(self, stream=None):
        hip_check(hip().hipEventRecord(self.h, stream.h if stream else None), "hipEventRecord")

    def elapsed_ms(self, end):
        hip_check(hip().hipEventSynchronize(end.h), "hipEventSynchronize")
        ms = C.c_float()
        hip_check(hip().hipEventElapsedTime(C.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value


def forward_host(ctx, layer, x, flags=0, with_state=True):
    """Run one layer on host activations through gmoe_forward_host; returns (x_out, state)."""
    lib = ctx.lib
    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0]
    s = ctx.shape
    out = np.empty_like(x)
    st = None
    state_p = None
    if with_state:
        st = {
            "xn": np.zeros((T, s.D), np.float32),
            "router_prob": np.zeros((T, s.E), np.float32),
            "topk_idx": np.zeros((T, s.K), np.int32),
            "topk_w": np.zeros((T, s.K), np.float32),
            "shared_out": np.zeros((T, s.D), np.float32),
            "routed_out": np.zeros((T, s.D), np.float32),
            "expert_offsets": np.zeros(s.E + 1, np.int32),
            "expert_tokens": np.zeros(max(1, T * s.K), np.int32),
        }
        state_p = C.byref(GmoeLayerState(*[ptr(st[n]) for n, _ in GmoeLayerState._fields_]))
    check(lib.gmoe_forward_host(ctx.h, layer, T, ptr(x), ptr(out), flags, state_p), "gmoe_forward_host")
    if st is not None:
        n = int(st["expert_offsets"][-1])
        st["expert_tokens"] = st["expert_tokens"][:n]
    return out, st
