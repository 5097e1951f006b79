"""Host-side mirror of the reference's GPU model context over the C-ABI.

``Model`` stands where GpuModelContext (src/gpu/model_gpu.zig:30-216) stands:
``Model.create`` ingests bf16 LayerWeights, ``forward_token`` is
gpuDispatchForwardToken (src/gpu/model_dispatch.zig:128-153),
``prefill_batch`` is gpuDispatchPrefillBatch (src/gpu/batch_dispatch.zig:
27-172), and ``kv_read`` / ``kv_write`` / ``read_state`` replace the UMA
slices the reference's host code reads and writes directly.
"""
import ctypes

import numpy as np

from ._abi import ChannelError, c_f32, c_u32, c_void_p, lib

MAX_SLOTS = 4096


class ModelConfig(ctypes.Structure):
    """chn_model_config: ModelConfig (src/model/types.zig:43-61) fields the GPU path uses."""
    _fields_ = [
        ("hidden_size", c_u32), ("intermediate_size", c_u32), ("vocab_size", c_u32),
        ("num_layers", c_u32), ("num_heads", c_u32), ("num_kv_heads", c_u32),
        ("head_dim", c_u32), ("rotary_dim", c_u32),
        ("global_head_dim", c_u32), ("num_global_kv_heads", c_u32),
        ("rms_norm_eps", c_f32), ("rope_theta", c_f32), ("rope_theta_full", c_f32),
        ("sliding_window", c_u32), ("k_eq_v", c_u32), ("max_prefill_tokens", c_u32),
        ("layer_full", ctypes.c_uint8 * 64),
        ("quiescence_thresh", c_f32), ("prefill_window", c_u32),
    ]
    _OPTIONAL = ("global_head_dim", "num_global_kv_heads", "quiescence_thresh", "prefill_window")

    @classmethod
    def from_dict(cls, d):
        c = cls()
        for name, _ in cls._fields_:
            if name == "layer_full":
                for i, v in enumerate(d["layer_full"]):
                    c.layer_full[i] = 1 if v else 0
            else:
                setattr(c, name, d.get(name, 0) if name in cls._OPTIONAL else d[name])
        return c

    def to_dict(self):
        d = {name: getattr(self, name) for name, _ in self._fields_ if name != "layer_full"}
        d["layer_full"] = [int(self.layer_full[i]) for i in range(self.num_layers)]
        return d


_U16P = ctypes.POINTER(ctypes.c_uint16)
_TENSORS = ("input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm",
            "post_attention_layernorm", "pre_feedforward_layernorm", "gate_proj", "up_proj",
            "down_proj", "post_feedforward_layernorm")


class LayerWeights(ctypes.Structure):
    """chn_layer_weights: LayerWeights (src/model/types.zig:13-41) as bf16 host pointers."""
    _fields_ = [(n, _U16P) for n in _TENSORS] + [("layer_scalar", c_f32), ("has_layer_scalar", ctypes.c_int)]


def _bf16_ptr(a, keep):
    if a is None:
        return None
    arr = np.ascontiguousarray(a, dtype=np.uint16)
    keep.append(arr)
    return arr.ctypes.data_as(_U16P)


_PROGRESS = ctypes.CFUNCTYPE(None, ctypes.c_size_t, ctypes.c_size_t, c_void_p)


class RingState(ctypes.Structure):
    """chn_ring_state: the DynamicRingBuffer state (src/ring_buffer.zig:17-355)
    that decides a contiguous history's slot lists."""
    _fields_ = [("num_anchors", c_u32), ("num_boundaries", c_u32), ("boundaries", c_void_p),
                ("recall_clocks", c_void_p)]


class Model:
    """A model resident in HBM: Q4 layer weights, Q8 tied embedding, 4096-slot
    fp32 KV caches per layer, the recorded decode graphs."""

    def __init__(self, ctx, handle):
        self.ctx = ctx
        self.handle = handle
        cfg = ModelConfig()
        self._check("chn_model_get_config", lib.chn_model_get_config(handle, ctypes.byref(cfg)))
        self.config = cfg
        self.H = cfg.hidden_size

    def _check(self, fn, rc):
        if rc != 0:
            raise ChannelError(fn, rc, lib.chn_last_error(self.ctx.handle).decode())

    @classmethod
    def create(cls, ctx, config, layers, embed_bf16, final_norm_bf16=None):
        """GpuModelContext.init: ``layers`` is a list of dicts keyed by the
        LayerWeights tensor names (bf16 as uint16 arrays; missing keys read as
        absent) plus an optional float ``layer_scalar``."""
        cfg = config if isinstance(config, ModelConfig) else ModelConfig.from_dict(config)
        keep = []
        arr = (LayerWeights * len(layers))()
        for i, l in enumerate(layers):
            for n in _TENSORS:
                setattr(arr[i], n, _bf16_ptr(l.get(n), keep))
            if l.get("layer_scalar") is not None:
                arr[i].layer_scalar = float(l["layer_scalar"])
                arr[i].has_layer_scalar = 1
        emb = np.ascontiguousarray(embed_bf16, dtype=np.uint16)
        fin = None if final_norm_bf16 is None else np.ascontiguousarray(final_norm_bf16, dtype=np.uint16)
        h = c_void_p()
        rc = lib.chn_model_create(ctx.handle, ctypes.byref(cfg), arr, emb.ctypes.data_as(c_void_p),
                                  None if fin is None else fin.ctypes.data_as(c_void_p), ctypes.byref(h))
        if rc != 0:
            raise ChannelError("chn_model_create", rc, lib.chn_last_error(ctx.handle).decode())
        return cls(ctx, h.value)

    @classmethod
    def synthetic(cls, ctx, config, seed):
        """Seeded synthetic weights generated in HBM (benchmarks)."""
        cfg = config if isinstance(config, ModelConfig) else ModelConfig.from_dict(config)
        h = c_void_p()
        rc = lib.chn_model_create_synthetic(ctx.handle, ctypes.byref(cfg), int(seed), ctypes.byref(h))
        if rc != 0:
            raise ChannelError("chn_model_create_synthetic", rc, lib.chn_last_error(ctx.handle).decode())
        return cls(ctx, h.value)

    def set_graph(self, enabled):
        """Replay the recorded decode graph (default) or launch its kernels
        one by one."""
        self._check("chn_model_set_graph", lib.chn_model_set_graph(self.handle, 1 if enabled else 0))

    @staticmethod
    def _slots(s):
        a = np.ascontiguousarray(s if s is not None else [], dtype=np.uint32)
        return a, (a.ctypes.data_as(c_void_p) if a.size else None)

    def forward_token(self, x, clock, slot_idx, active_slots, sliding_slots, topk=True):
        """gpuDispatchForwardToken: returns (token, ids, vals); ids/vals are
        None without topk (the no-logits graph, the reference's prefill
        command buffer)."""
        xx = np.ascontiguousarray(x, dtype=np.float32)
        if xx.size != self.H:
            raise ValueError(f"x has {xx.size} elements, hidden_size is {self.H}")
        a, ap = self._slots(active_slots)
        s, sp = self._slots(sliding_slots)
        ids = np.zeros(64, np.uint32) if topk else None
        vals = np.zeros(64, np.float32) if topk else None
        tok = c_u32()
        self._check("chn_decode_step", lib.chn_decode_step(
            self.handle, xx.ctypes.data_as(c_void_p), int(clock), int(slot_idx), ap, a.size, sp, s.size,
            None if ids is None else ids.ctypes.data_as(c_void_p),
            None if vals is None else vals.ctypes.data_as(c_void_p), ctypes.byref(tok)))
        return tok.value, ids, vals

    def forward_token_id(self, token, clock, slot_idx, active_slots, sliding_slots, topk=True):
        """Embedding gather on the device, then forward_token."""
        a, ap = self._slots(active_slots)
        s, sp = self._slots(sliding_slots)
        ids = np.zeros(64, np.uint32) if topk else None
        vals = np.zeros(64, np.float32) if topk else None
        tok = c_u32()
        self._check("chn_decode_token", lib.chn_decode_token(
            self.handle, int(token), int(clock), int(slot_idx), ap, a.size, sp, s.size,
            None if ids is None else ids.ctypes.data_as(c_void_p),
            None if vals is None else vals.ctypes.data_as(c_void_p), ctypes.byref(tok)))
        return tok.value, ids, vals

    def decode_greedy(self, token, clock, n_steps, num_anchors=0, boundaries=(), recall_clocks=None):
        """n_steps greedy steps on the device over the reference's 4096-slot
        ring (chn_ring_state: anchors, turn boundaries oldest first, the
        clocks of the 128 recall slots or None); returns the generated ids."""
        out = np.zeros(max(int(n_steps), 1), np.uint32)
        b = np.ascontiguousarray(boundaries, dtype=np.uint32)
        rc = None if recall_clocks is None else np.ascontiguousarray(recall_clocks, dtype=np.uint32)
        if rc is not None and rc.size != 128:
            raise ValueError("recall_clocks must hold 128 entries")
        st = RingState(int(num_anchors), b.size, b.ctypes.data_as(c_void_p) if b.size else None,
                       None if rc is None else rc.ctypes.data_as(c_void_p))
        self._check("chn_decode_greedy", lib.chn_decode_greedy(self.handle, int(token), int(clock), int(n_steps),
                                                               ctypes.byref(st), out.ctypes.data_as(c_void_p)))
        return out[: int(n_steps)]

    def prefill_batch(self, tokens, slots, start_clock, num_prev_slots, embed_bf16=None,
                      logits=True, topk=True, progress=None):
        """gpuDispatchPrefillBatch: returns (logits or None, ids or None, vals or None)."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        sl = np.ascontiguousarray(slots, dtype=np.uint32)
        emb = None if embed_bf16 is None else np.ascontiguousarray(embed_bf16, dtype=np.uint16)
        lg = np.zeros(self.config.vocab_size, np.float32) if logits else None
        ids = np.zeros(64, np.uint32) if topk else None
        vals = np.zeros(64, np.float32) if topk else None
        cb = _PROGRESS(lambda i, n, _c: progress(i, n)) if progress else None
        p = lambda a: None if a is None else a.ctypes.data_as(c_void_p)  # noqa: E731
        self._check("chn_prefill", lib.chn_prefill(
            self.handle, p(t), t.size, p(emb), p(sl), sl.size, int(start_clock), int(num_prev_slots),
            p(lg), p(ids), p(vals), cb, None))
        return lg, ids, vals

    def layer_kv_dim(self, layer):
        c = self.config
        full = bool(c.layer_full[layer])
        D = c.global_head_dim if full and c.global_head_dim else c.head_dim
        nkv = c.num_global_kv_heads if full and c.num_global_kv_heads else c.num_kv_heads
        return D * nkv

    def kv_read(self, layer, slot_begin, n):
        kvd = self.layer_kv_dim(layer)
        k = np.zeros((n, kvd), np.float32)
        v = np.zeros((n, kvd), np.float32)
        self._check("chn_kv_read", lib.chn_kv_read(self.handle, layer, slot_begin, n,
                                                   k.ctypes.data_as(c_void_p), v.ctypes.data_as(c_void_p)))
        return k, v

    def kv_write(self, layer, slot_begin, k, v):
        kvd = self.layer_kv_dim(layer)
        kk = np.ascontiguousarray(k, dtype=np.float32).reshape(-1, kvd)
        vv = np.ascontiguousarray(v, dtype=np.float32).reshape(-1, kvd)
        if kk.shape != vv.shape:
            raise ValueError("k and v differ in shape")
        self._check("chn_kv_write", lib.chn_kv_write(self.handle, layer, slot_begin, kk.shape[0],
                                                     kk.ctypes.data_as(c_void_p), vv.ctypes.data_as(c_void_p)))

    def read_state(self):
        """(x, normed_x): the hidden state and last normed row."""
        x = np.zeros(self.H, np.float32)
        nx = np.zeros(self.H, np.float32)
        self._check("chn_model_read_state", lib.chn_model_read_state(
            self.handle, x.ctypes.data_as(c_void_p), nx.ctypes.data_as(c_void_p)))
        return x, nx

    def read_logits(self):
        """The fp32 logits of the last step or prefill that computed them."""
        lg = np.zeros(self.config.vocab_size, np.float32)
        self._check("chn_model_read_logits", lib.chn_model_read_logits(self.handle, lg.ctypes.data_as(c_void_p)))
        return lg

    def replay(self, with_logits=True):
        """submitPreRecorded(cmd_buf_decode): the recorded step once more on
        the inputs already on the device; returns (ids, vals) or None."""
        ids = np.zeros(64, np.uint32) if with_logits else None
        vals = np.zeros(64, np.float32) if with_logits else None
        self._check("chn_model_replay", lib.chn_model_replay(
            self.handle, 1 if with_logits else 0, None if ids is None else ids.ctypes.data_as(c_void_p),
            None if vals is None else vals.ctypes.data_as(c_void_p)))
        return (ids, vals) if with_logits else None

    def close(self):
        if self.handle is not None:
            lib.chn_model_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
