"""ctypes mirror of include/glm_model.h (glm.c's model.h:7-164) and a driver for the
--backend hip drop-in (include/glm_backend.h, libglm_hip.so).

GlmModel builds the Runtime / RunState pair that glm.c hands its backend: a
checkpoint view whose MoE layers point at HostLayer arrays (LayerMoeShared and
LayerMoeRouted per layer, model.h:65-84, indexed 1..n_layers-1 as infer.c:668,717
fill them) and the decode-time RunState buffers the MoE layer reads and writes
(model.h:132-159). It is plumbing for tests and the benchmark: every computation
goes through libglm_hip.so's C entry points.
"""
import ctypes as C

import numpy as np

import gmoe

BACKEND_CPU, BACKEND_METAL, BACKEND_HIP = 0, 1, 2

_i32, _u32, _u64, _P = C.c_int32, C.c_uint32, C.c_uint64, C.c_void_p


class RuntimeConfig(C.Structure):
    _fields_ = [("magic", _u32), ("version", _u32), ("dim", _i32), ("hidden_dim", _i32), ("n_layers", _i32),
                ("n_heads", _i32), ("n_kv_heads", _i32), ("vocab_size", _i32), ("seq_len", _i32), ("rope_dim", _i32),
                ("q_lora_rank", _i32), ("kv_lora_rank", _i32), ("kv_mqa_width", _i32), ("n_routed_experts", _i32),
                ("n_experts_used", _i32), ("n_shared_experts", _i32), ("bos_id", _i32), ("eos_id", _i32),
                ("group_size", _u64), ("off_norm", _u64), ("off_tok_q", _u64), ("off_tok_s", _u64),
                ("off_out_q", _u64), ("off_out_s", _u64), ("total_bytes", _u64), ("off_l0_ffn_norm", _u64),
                ("off_l0_ffn_gate_q", _u64), ("off_l0_ffn_gate_s", _u64), ("off_l0_ffn_up_q", _u64),
                ("off_l0_ffn_up_s", _u64), ("off_l0_ffn_down_q", _u64), ("off_l0_ffn_down_s", _u64),
                ("l0_qk_nope_dim", _i32), ("l0_head_k_dim", _i32), ("l0_v_head_dim", _i32), ("l0_flags", _i32),
                ("moe_ffn_dim", _i32)]


class LayerAttnWeights(C.Structure):
    _fields_ = [(n, _P) for n in ("attn_norm", "q_a_norm", "kv_a_norm", "q_a_q", "q_a_s", "q_b_q", "q_b_s", "kv_a_q",
                                  "kv_a_s", "k_b_q", "k_b_s", "v_b_q", "v_b_s", "attn_out_q", "attn_out_s")]


SHARED_FIELDS = ("ffn_norm", "gate_inp", "exp_probs_b", "gate_sh_q", "gate_sh_s", "up_sh_q", "up_sh_s", "down_sh_q",
                 "down_sh_s")
ROUTED_FIELDS = ("gate_q", "gate_s", "up_q", "up_s", "down_q", "down_s")


class LayerMoeShared(C.Structure):
    _fields_ = [(n, _P) for n in SHARED_FIELDS]


class LayerMoeRouted(C.Structure):
    _fields_ = [(n, _P) for n in ROUTED_FIELDS]


class Runtime(C.Structure):
    _fields_ = ([("cfg", RuntimeConfig), ("data", _P), ("file_size", C.c_size_t)]
                + [(n, _P) for n in ("output_norm", "tok_q", "tok_s", "out_q", "out_s")]
                + [("has_l0_ffn", C.c_int)]
                + [(n, _P) for n in ("l0_ffn_norm", "l0_ffn_gate_q", "l0_ffn_gate_s", "l0_ffn_up_q", "l0_ffn_up_s",
                                     "l0_ffn_down_q", "l0_ffn_down_s")]
                + [("has_l0_attn", C.c_int)]
                + [(n, _P) for n in ("l0_attn_norm", "l0_q_a_norm", "l0_kv_a_norm", "l0_q_a_q", "l0_q_a_s", "l0_q_b_q",
                                     "l0_q_b_s", "l0_kv_a_q", "l0_kv_a_s", "l0_k_b_q", "l0_k_b_s", "l0_v_b_q",
                                     "l0_v_b_s", "l0_attn_out_q", "l0_attn_out_s")]
                + [("has_all_attn", C.c_int), ("attn_layers", C.POINTER(LayerAttnWeights)),
                   ("has_moe_shared", C.c_int), ("moe_layers", C.POINTER(LayerMoeShared)),
                   ("has_moe_routed", C.c_int), ("moe_routed_layers", C.POINTER(LayerMoeRouted))])


class RunState(C.Structure):
    _fields_ = ([(n, _P) for n in ("x", "xn", "xb", "ff_gate", "ff_up", "logits")]
                + [("cache_cap", C.c_int), ("n_attn_layers", C.c_int)]
                + [(n, _P) for n in ("k_cache_comp", "k_cache_pe", "q_a", "q_full", "kv_a", "q_nope", "q_pe", "q_abs",
                                     "att_scores", "att_ctx", "att_concat", "moe_gate", "moe_up", "moe_router",
                                     "moe_out_acc", "moe_topk_idx", "moe_topk_w")])


STRUCTS = {"RuntimeConfig": RuntimeConfig, "LayerAttnWeights": LayerAttnWeights, "LayerMoeShared": LayerMoeShared,
           "LayerMoeRouted": LayerMoeRouted, "Runtime": Runtime, "RunState": RunState}


def backend_lib():
    lib = gmoe.host_lib()
    if not getattr(lib, "_backend_typed", False):
        RP, SP = C.POINTER(Runtime), C.POINTER(RunState)
        lib.glm_backend_init.argtypes = [C.c_int, RP, SP]
        lib.glm_backend_init.restype = C.c_int
        lib.glm_backend_free.argtypes = [C.c_int]
        lib.glm_backend_free.restype = None
        lib.glm_backend_try_hip_moe.argtypes = [RP, SP, C.c_int, C.c_int]
        lib.glm_backend_try_hip_moe.restype = C.c_int
        lib.glm_backend_forward_token.argtypes = [C.c_int, RP, SP, C.c_int, C.c_int, C.c_int]
        lib.glm_backend_forward_token.restype = C.c_int
        lib._backend_typed = True
    return lib


class CkptSpec(C.Structure):
    """glm_ckpt_spec (include/glm_ckpt.h): shape and draws of a synthetic v4 checkpoint."""
    _fields_ = ([(n, C.c_int32) for n in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size",
                                          "seq_len", "rope_dim", "q_lora_rank", "kv_lora_rank", "n_routed_experts",
                                          "n_experts_used", "bos_id", "eos_id", "qk_nope_dim", "v_head_dim",
                                          "moe_ffn_dim", "group_size")]
                + [("seed", C.c_uint64)]
                + [(n, C.c_int32) for n in ("norm_mode", "bias_mode", "scale_mode")])


def ckpt_lib():
    lib = gmoe.host_lib()
    if not getattr(lib, "_ckpt_typed", False):
        RP = C.POINTER(Runtime)
        lib.glm_ckpt_write_synth.argtypes = [C.c_char_p, C.POINTER(CkptSpec)]
        lib.glm_ckpt_write_synth.restype = C.c_int
        lib.glm_ckpt_open.argtypes = [C.c_char_p, RP]
        lib.glm_ckpt_open.restype = C.c_int
        lib.glm_ckpt_close.argtypes = [RP]
        lib.glm_ckpt_close.restype = None
        lib.glm_ckpt_error.argtypes = []
        lib.glm_ckpt_error.restype = C.c_char_p
        lib.glm_ckpt_layout.argtypes = [RP, C.POINTER(C.c_uint64), C.c_int]
        lib.glm_ckpt_layout.restype = C.c_int
        lib._ckpt_typed = True
    return lib


def write_synth_checkpoint(path, spec):
    """glm_ckpt_write_synth: a synthetic v4 .bin of this CkptSpec at path."""
    lib = ckpt_lib()
    if lib.glm_ckpt_write_synth(str(path).encode(), C.byref(spec)) != 0:
        raise RuntimeError(f"glm_ckpt_write_synth: {lib.glm_ckpt_error().decode()}")


class Checkpoint:
    """A v4 .bin mapped by glm_ckpt_open: its Runtime, as glm.c's runtime_open fills it."""

    def __init__(self, path):
        self.lib = ckpt_lib()
        self.rt = Runtime()
        if self.lib.glm_ckpt_open(str(path).encode(), C.byref(self.rt)) != 0:
            raise RuntimeError(f"glm_ckpt_open: {self.lib.glm_ckpt_error().decode()}")

    def layout(self):
        n = self.lib.glm_ckpt_layout(C.byref(self.rt), None, 0)
        out = (C.c_uint64 * n)()
        self.lib.glm_ckpt_layout(C.byref(self.rt), out, n)
        return np.frombuffer(out, np.uint64).copy()

    def close(self):
        if self.rt.data:
            self.lib.glm_ckpt_close(C.byref(self.rt))


class GlmModel:
    """A glm.c Runtime and a RunState sized for one decode token. The Runtime's MoE layers
    1..len(layers) are the given HostLayers (layer 0 has no MoE block, as in
    GLM-4.7-Flash), or it is a Checkpoint's."""

    def __init__(self, shape, layers=None, checkpoint=None):
        self.shape = shape
        if checkpoint is not None:
            self.ckpt = checkpoint  # keeps the mapping alive
            self.rt = checkpoint.rt
            self._state(shape)
            return
        self.layers = list(layers)  # keep the arrays alive
        n_layers = len(self.layers) + 1
        cfg = RuntimeConfig()
        cfg.dim, cfg.n_layers, cfg.moe_ffn_dim = shape.D, n_layers, shape.F
        cfg.n_routed_experts, cfg.n_experts_used, cfg.n_shared_experts = shape.E, shape.K, 1
        cfg.group_size = shape.gs
        self.shared = (LayerMoeShared * n_layers)()
        self.routed = (LayerMoeRouted * n_layers)()
        for l, hl in enumerate(self.layers, start=1):
            for n in SHARED_FIELDS:
                setattr(self.shared[l], n, gmoe.ptr(getattr(hl, n)))
            for n in ROUTED_FIELDS:
                setattr(self.routed[l], n, gmoe.ptr(getattr(hl, n)))
        rt = Runtime()
        rt.cfg = cfg
        rt.has_moe_shared = 1
        rt.moe_layers = C.cast(self.shared, C.POINTER(LayerMoeShared))
        rt.has_moe_routed = 1
        rt.moe_routed_layers = C.cast(self.routed, C.POINTER(LayerMoeRouted))
        self.rt = rt
        self._state(shape)

    def _state(self, shape):
        D, E, K = shape.D, shape.E, shape.K
        self.buf = {"x": np.zeros(D, np.float32), "xn": np.zeros(D, np.float32), "xb": np.zeros(D, np.float32),
                    "moe_router": np.zeros(E, np.float32), "moe_out_acc": np.zeros(D, np.float32),
                    "moe_topk_idx": np.zeros(K, np.int32), "moe_topk_w": np.zeros(K, np.float32)}
        st = RunState()
        for n, a in self.buf.items():
            setattr(st, n, gmoe.ptr(a))
        self.st = st

    def init(self, backend=BACKEND_HIP):
        """glm_backend_init (backend.h:7): uploads every MoE layer; exits the process on failure."""
        return backend_lib().glm_backend_init(backend, C.byref(self.rt), C.byref(self.st))

    def try_moe(self, layer, debug=0):
        """glm_backend_try_hip_moe: 0 if the GPU ran the layer on the RunState, else -1."""
        return backend_lib().glm_backend_try_hip_moe(C.byref(self.rt), C.byref(self.st), layer, debug)

    def free(self, backend=BACKEND_HIP):
        backend_lib().glm_backend_free(backend)


def forward_lib():
    """libglm_hip.so's token forward (include/glm_forward.h)."""
    lib = backend_lib()
    if not getattr(lib, "_forward_typed", False):
        RP, SP, FP, IP = C.POINTER(Runtime), C.POINTER(RunState), C.POINTER(C.c_float), C.POINTER(C.c_int)
        lib.glm_runstate_build.argtypes = [SP, RP, C.c_int]
        lib.glm_runstate_build.restype = C.c_int
        lib.glm_runstate_free.argtypes = [SP]
        lib.glm_runstate_free.restype = None
        lib.glm_hip_forward_token.argtypes = [RP, SP, C.c_int, C.c_int, C.c_int]
        lib.glm_hip_forward_token.restype = C.c_int
        lib.glm_hip_forward_token_dual_checkpoints.argtypes = [RP, SP, C.c_int, C.c_int, C.c_int, FP, C.c_int, C.c_int,
                                                               IP, FP, C.c_int, C.c_int, IP]
        lib.glm_hip_forward_token_dual_checkpoints.restype = C.c_int
        lib.glm_argmax.argtypes = [FP, C.c_int]
        lib.glm_argmax.restype = C.c_int
        lib.glm_hip_model_active.argtypes = []
        lib.glm_hip_model_active.restype = C.c_int
        lib.glm_hip_prefill.argtypes = [RP, SP, IP, C.c_int, C.c_int, C.c_int]
        lib.glm_hip_prefill.restype = C.c_int
        lib.glm_hip_model_read_cache.argtypes = [C.c_int, C.c_int, C.c_int, FP, FP]
        lib.glm_hip_model_read_cache.restype = C.c_int
        lib.glm_hip_model_forward.argtypes = [RP, SP, C.c_int, C.c_int, C.c_int, FP, FP, FP]
        lib.glm_hip_model_forward.restype = C.c_int
        lib._forward_typed = True
    return lib


class Decoder:
    """glm.c's decode state on a Checkpoint: a RunState from glm_runstate_build with a
    latent cache of cache_cap positions, advanced one token at a time by
    glm_hip_forward_token (the MoE layers on the GPU after glm_backend_init(BACKEND_HIP),
    which a checkpoint without MoE layers does not need)."""

    def __init__(self, checkpoint, cache_cap):
        self.lib = forward_lib()
        self.ckpt = checkpoint
        self.rt = checkpoint.rt
        self.st = RunState()
        if self.lib.glm_runstate_build(C.byref(self.st), C.byref(self.rt), cache_cap) != 0:
            raise RuntimeError("glm_runstate_build failed")
        c = self.rt.cfg
        self.L, self.D, self.V = c.n_layers, c.dim, c.vocab_size
        self.backend = BACKEND_CPU
        if self.rt.has_moe_shared and c.n_layers > 1:
            self.backend = self.lib.glm_backend_init(BACKEND_HIP, C.byref(self.rt), C.byref(self.st))

    def logits(self):
        return np.ctypeslib.as_array(C.cast(self.st.logits, C.POINTER(C.c_float)), shape=(self.V,)).copy()

    def step(self, token, pos, checkpoints=False):
        """One token at position pos; returns the logits, and with checkpoints also x after
        each layer's attention and after its FFN ([n_layers][dim] each) from
        glm_hip_forward_token_dual_checkpoints on the state before the step."""
        FP = C.POINTER(C.c_float)
        attn = layer = None
        if checkpoints:
            attn = np.zeros((self.L, self.D), np.float32)
            layer = np.zeros((self.L, self.D), np.float32)
            na, nl = C.c_int(), C.c_int()
            rc = self.lib.glm_hip_forward_token_dual_checkpoints(
                C.byref(self.rt), C.byref(self.st), token, pos, 0, attn.ctypes.data_as(FP), self.D, self.L,
                C.byref(na), layer.ctypes.data_as(FP), self.D, self.L, C.byref(nl))
            if rc != 0:
                raise RuntimeError(f"glm_hip_forward_token_dual_checkpoints failed at pos {pos}")
        if self.lib.glm_hip_forward_token(C.byref(self.rt), C.byref(self.st), token, pos, 0) != 0:
            raise RuntimeError(f"glm_hip_forward_token failed at pos {pos}")
        out = self.logits()
        return (out, attn, layer) if checkpoints else out

    def prefill(self, tokens, pos0=0):
        """The prompt tokens at positions pos0.. (glm_hip_prefill: batches through the GPU
        model when it is active); returns the last token's logits."""
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        if toks.ndim != 1 or toks.size == 0:
            raise ValueError("prefill takes a non-empty 1-d sequence of tokens")
        rc = self.lib.glm_hip_prefill(C.byref(self.rt), C.byref(self.st), toks.ctypes.data_as(C.POINTER(C.c_int)),
                                      int(toks.size), int(pos0), 0)
        if rc != 0:
            raise RuntimeError(f"glm_hip_prefill failed at positions {pos0}..{pos0 + toks.size - 1}")
        return self.logits()

    def read_cache(self, layer, pos0, n, kv, rope):
        """Positions pos0..pos0+n-1 of the GPU model's latent cache of attention layer `layer`:
        (comp [n][kv], pe [n][rope])."""
        FP = C.POINTER(C.c_float)
        comp = np.zeros((n, kv), np.float32)
        pe = np.zeros((n, rope), np.float32)
        if self.lib.glm_hip_model_read_cache(layer, pos0, n, comp.ctypes.data_as(FP), pe.ctypes.data_as(FP)) != 0:
            raise RuntimeError("glm_hip_model_read_cache failed")
        return comp, pe

    def on_gpu(self):
        """True when every step of the forward runs on the GPU model (gmoe_model.h)."""
        return self.backend == BACKEND_HIP and bool(self.lib.glm_hip_model_active())

    def argmax(self):
        return self.lib.glm_argmax(C.cast(self.st.logits, C.POINTER(C.c_float)), self.V)

    def free(self):
        if self.backend == BACKEND_HIP:
            self.lib.glm_backend_free(BACKEND_HIP)
            self.backend = BACKEND_CPU
        if self.st.x:
            self.lib.glm_runstate_free(C.byref(self.st))


def write_tokenizer(path, vocab_size, bos_id, eos_id):
    """A `.tokenizer` sidecar in the layout glm.c's loader reads (infer.c:232-285): max token
    length, bos and eos ids (u32 each), then per token a float score, a u32 length and the
    bytes. Tokens 33..126 are those single printable ASCII bytes (so a prompt of such bytes
    encodes to one token per byte, infer.c:1328-1366, with no merges); every other token i is
    the text "<t{i}>". For glm.c's app on synthetic checkpoints."""
    import struct
    toks = [bytes([i]) if 33 <= i < 127 else f"<t{i}>".encode() for i in range(vocab_size)]
    with open(path, "wb") as f:
        f.write(struct.pack("<III", max(len(t) for t in toks), bos_id, eos_id))
        for t in toks:
            f.write(struct.pack("<fI", 0.0, len(t)))
            f.write(t)
