"""A whole decode step on the device: the reference's `LlamaBackend::logits_batch`
(garuda/src/llama/mod.rs:1134-1206) for its decode case, every sequence taking one new
token, over gmoe_model_* (include/garuda_moe.h).

`DecodeModel` holds the model's weights as the library's registered objects (one
`MoeLayer` and four `DenseWeight` projections per layer, the output head as a
`DenseWeight`, the paged `KvCache`) plus the norm weights and the f32 token table. Each
`decode_step(seqs, tokens)` embeds the tokens, runs every layer as `layer_batch_over`
does (llama/mod.rs:851-893), applies the output norm and head, and returns the greedy
next tokens (runtime/mod.rs:98-105) and, on request, the logits.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import lib
from .moe import _check, _fp


class GmoeModelDesc(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("d_model", C.c_uint32), ("vocab", C.c_uint32), ("rms_eps", C.c_float),
                ("kv", C.c_void_p), ("moe_layers", C.POINTER(C.c_uint32)), ("wq", C.POINTER(C.c_uint32)),
                ("wk", C.POINTER(C.c_uint32)), ("wv", C.POINTER(C.c_uint32)), ("wo", C.POINTER(C.c_uint32)),
                ("output", C.c_uint32), ("attn_norm", C.POINTER(C.c_float)), ("ffn_norm", C.POINTER(C.c_float)),
                ("output_norm", C.POINTER(C.c_float)), ("token_embd_qtype", C.c_uint32),
                ("token_embd", C.c_void_p), ("output_math", C.c_uint32)]

OUTPUT_TIED = 0xFFFFFFFF


def _u32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32).reshape(-1))


class DecodeModel:
    """moe_layers / wq / wk / wv / wo: per layer, the registered MoeLayer and DenseWeight
    objects; output: the head's DenseWeight, or None when the checkpoint ties the head to
    the token table (llama/mod.rs:565-571; output_math then sets its arithmetic); kv: a
    KvCache of n_layers layers; attn_norm / ffn_norm: [n_layers, d]; output_norm: [d];
    token_embd: [vocab, d] f32, or (qtype, packed rows, vocab, d) to keep the table packed in
    HBM, a row dequantised per token (Weight::row, llama/mod.rs:198-212). The objects must
    outlive the model (it keeps their ids, not copies)."""

    def __init__(self, dev, kv, moe_layers, wq, wk, wv, wo, output, attn_norm, ffn_norm, output_norm, token_embd,
                 rms_eps: float = 1e-5, output_math: int = 0):
        n_layers = len(moe_layers)
        if isinstance(token_embd, tuple):
            embd_qt, raw, vocab, d = token_embd
            table = np.ascontiguousarray(raw, dtype=np.uint8)
        else:
            table = np.ascontiguousarray(token_embd, dtype=np.float32)
            embd_qt = 0
            vocab, d = table.shape
        self.dev, self.kv, self.n_layers, self.d, self.vocab = dev, kv, n_layers, d, vocab
        self._keep = (moe_layers, wq, wk, wv, wo, output)
        ids = {name: _u32([o.id for o in objs]) for name, objs in
               (("moe", moe_layers), ("wq", wq), ("wk", wk), ("wv", wv), ("wo", wo))}
        an = np.ascontiguousarray(attn_norm, dtype=np.float32).reshape(n_layers, d)
        fn = np.ascontiguousarray(ffn_norm, dtype=np.float32).reshape(n_layers, d)
        on = np.ascontiguousarray(output_norm, dtype=np.float32).reshape(d)
        u32p = C.POINTER(C.c_uint32)
        desc = GmoeModelDesc(n_layers, d, vocab, rms_eps, kv._h,
                             ids["moe"].ctypes.data_as(u32p), ids["wq"].ctypes.data_as(u32p),
                             ids["wk"].ctypes.data_as(u32p), ids["wv"].ctypes.data_as(u32p),
                             ids["wo"].ctypes.data_as(u32p), OUTPUT_TIED if output is None else output.id,
                             _fp(an), _fp(fn), _fp(on), embd_qt, table.ctypes.data, output_math)
        h = C.c_void_p()
        _check(lib().gmoe_model_create(dev.handle, C.byref(desc), C.byref(h)))
        self._h = h

    def decode_step(self, seqs, tokens, want_logits: bool = False):
        """Greedy next token of each sequence (and [n, vocab] logits if asked)."""
        seqs, tokens = _u32(seqs), _u32(tokens)
        n = seqs.size
        if tokens.size != n:
            raise ValueError("one token per sequence")
        nxt = np.zeros(n, dtype=np.uint32)
        logits = np.empty((n, self.vocab), dtype=np.float32) if want_logits else None
        u32p = C.POINTER(C.c_uint32)
        _check(lib().gmoe_model_decode(self._h, n, seqs.ctypes.data_as(u32p), tokens.ctypes.data_as(u32p),
                                       nxt.ctypes.data_as(u32p), _fp(logits) if logits is not None else None))
        return (nxt, logits) if want_logits else nxt

    def prefill(self, seq: int, tokens, n_last: int = 1, want_logits: bool = False):
        """A prompt through the model (gmoe_model_prefill, forward_tail + logits_multi):
        the tokens take the sequence's next positions, in chunks of 256 run layer-major;
        the greedy next token after each of the last n_last positions (and their [n_last,
        vocab] logits if asked)."""
        tokens = _u32(tokens)
        nxt = np.zeros(n_last, dtype=np.uint32)
        logits = np.empty((n_last, self.vocab), dtype=np.float32) if want_logits else None
        u32p = C.POINTER(C.c_uint32)
        _check(lib().gmoe_model_prefill(self._h, seq, tokens.size, tokens.ctypes.data_as(u32p), n_last,
                                        nxt.ctypes.data_as(u32p), _fp(logits) if logits is not None else None))
        return (nxt, logits) if want_logits else nxt

    def set_graphs(self, enable: bool) -> None:
        """Replay decode steps from a HIP graph (the default) or issue every launch of every
        step (gmoe_model_set_graphs)."""
        _check(lib().gmoe_model_set_graphs(self._h, 1 if enable else 0))

    def graph_ready(self, n: int) -> bool:
        """Whether a graph of the step at batch size n is held."""
        return bool(lib().gmoe_model_graph_ready(self._h, n))

    TRACE_KEYS = ("x", "h_attn", "q", "k", "v", "context", "attn_out", "x_mid", "h_ffn", "moe_out")

    def decode_step_trace(self, seqs, tokens):
        """decode_step that also returns every layer's activations (gmoe_model_decode_trace):
        (next, logits, layers, final), layers[l] a dict of TRACE_KEYS -> [n, width] arrays,
        final a dict of x (the last residual) and h (its output norm)."""
        seqs, tokens = _u32(seqs), _u32(tokens)
        n = seqs.size
        if tokens.size != n:
            raise ValueError("one token per sequence")
        nxt = np.zeros(n, dtype=np.uint32)
        logits = np.empty((n, self.vocab), dtype=np.float32)
        trace = np.empty(lib().gmoe_model_trace_floats(self._h, n), dtype=np.float32)
        u32p = C.POINTER(C.c_uint32)
        _check(lib().gmoe_model_decode_trace(self._h, n, seqs.ctypes.data_as(u32p), tokens.ctypes.data_as(u32p),
                                             nxt.ctypes.data_as(u32p), _fp(logits), _fp(trace)))
        qd, kvd, d = self.kv.n_heads * self.kv.hd, self.kv.kv_dim, self.d
        widths = (d, d, qd, kvd, kvd, qd, d, d, d, d)
        at, layers = 0, []
        for _ in range(self.n_layers):
            rec = {}
            for key, w in zip(self.TRACE_KEYS, widths):
                rec[key] = trace[at:at + n * w].reshape(n, w)
                at += n * w
            layers.append(rec)
        final = {"x": trace[at:at + n * d].reshape(n, d), "h": trace[at + n * d:at + 2 * n * d].reshape(n, d)}
        return nxt, logits, layers, final

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().gmoe_model_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
