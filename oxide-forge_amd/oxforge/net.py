"""ctypes bindings of include/oxforge_net.h (the executor entry points)."""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, byref, c_char_p, c_float, c_int, c_long, c_size_t, c_uint64, c_void_p

import numpy as np

from . import _lib
from ._lib import NULL_SLICE, Slice, call

TP_SLOTS = ["WQ", "BQ", "WK", "BK", "WV", "BV", "POS", "W1", "B1", "W2", "B2", "WO", "BO",
            "G1", "BE1", "G2", "BE2"]
ENCODER_INFERENCE, ENCODER_TRAINING, DECODER_INFERENCE = 0, 1, 2
RMS, LAYER = 0, 1
# forge_checkpoint_kind
(CK_LINEAR, CK_MLP_INFERENCE, CK_MLP_TRAINING, CK_ENCODER_INFERENCE, CK_ENCODER_TRAINING,
 CK_DECODER_INFERENCE) = range(6)


class TransformerDesc(ctypes.Structure):
    _fields_ = [("seq", c_size_t), ("hidden", c_size_t), ("ffn", c_size_t), ("out", c_size_t),
                ("norm_type", c_int), ("kind", c_int), ("qkv_streams", c_int),
                ("ffn_activation", c_int)]


SIGNATURES = {
    "forge_net_model_destroy": [c_void_p],
    "forge_net_linear_create": [c_void_p, Slice, c_size_t, c_size_t, Slice, c_int,
                                POINTER(c_void_p)],
    "forge_net_linear_forward": [c_void_p, Slice, c_size_t, Slice, Slice, Slice],
    "forge_net_linear_backward": [c_void_p, Slice, Slice, c_size_t, Slice, Slice],
    "forge_net_linear_input_gradient": [c_void_p, Slice, c_size_t, Slice],
    "forge_net_linear_learn": [c_void_p, Slice, Slice, Slice, c_size_t, c_float],
    "forge_net_linear_loss_rows": [c_void_p, Slice, Slice, c_size_t, c_size_t, Slice],
    "forge_net_linear_param": [c_void_p, c_int, POINTER(Slice)],
    "forge_net_mlp_create": [c_void_p, c_size_t, POINTER(c_size_t), POINTER(c_int), POINTER(Slice),
                             POINTER(Slice), c_long, c_long, c_int, POINTER(c_void_p)],
    "forge_net_mlp_forward": [c_void_p, Slice, c_size_t, Slice],
    "forge_net_mlp_backward": [c_void_p, Slice, c_size_t, c_float, Slice],
    "forge_net_mlp_param": [c_void_p, c_size_t, c_int, POINTER(Slice)],
    "forge_net_transformer_create": [c_void_p, POINTER(TransformerDesc), POINTER(Slice),
                                     POINTER(c_void_p)],
    "forge_net_transformer_forward": [c_void_p, Slice, Slice],
    "forge_net_transformer_backward": [c_void_p, Slice, c_float, Slice, POINTER(Slice)],
    "forge_net_transformer_param": [c_void_p, c_int, POINTER(Slice)],
    "forge_net_transformer_set_score_bytes": [c_void_p, c_size_t],
    "forge_net_transformer_set_fold_norms": [c_void_p, c_int],
    "forge_net_checkpoint_save": [c_void_p, c_char_p],
    "forge_net_checkpoint_load": [c_void_p, c_char_p, c_int, POINTER(c_void_p)],
    "forge_checkpoint_inspect": [c_char_p, c_char_p, c_size_t, POINTER(c_uint64)],
    "forge_net_model_dims": [c_void_p, POINTER(c_size_t), c_size_t, POINTER(c_size_t)],
    "forge_net_transformer_describe": [c_void_p, POINTER(TransformerDesc)],
}

_declared = False


def _declare():
    global _declared
    if _declared:
        return
    lib = _lib.load()
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = c_int
    _declared = True


def _sl(a):
    return NULL_SLICE if a is None else a.slice


def _read(rt, sl: Slice, shape):
    out = np.empty(shape, np.float32)
    if sl.ptr:
        call("forge_memcpy_d2h", rt.handle, out.ctypes.data_as(c_void_p), sl, out.size)
    return out


class _Model:
    def __init__(self, rt):
        _declare()
        self.rt = rt
        self.h = c_void_p()
        rt.adopt(self)

    def close(self):
        # A model must be destroyed before its runtime; Runtime.close()
        # closes its models first, so a model outliving it holds nothing.
        if self.h and self.rt.handle:
            call("forge_net_model_destroy", self.h)
        self.h = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def save(self, path):
        """dump_* (model.rs:53-207): writes <path>.toml and <path>.bin."""
        call("forge_net_checkpoint_save", self.h, os.fsencode(path))

    def _dims(self):
        cap = 64
        dims = (c_size_t * cap)()
        n = c_size_t()
        call("forge_net_model_dims", self.h, dims, cap, byref(n))
        if n.value > cap:
            dims = (c_size_t * n.value)()
            call("forge_net_model_dims", self.h, dims, n.value, byref(n))
        return [int(d) for d in dims[:n.value]]


class Linear(_Model):
    """Linear (linear.rs:72-532) on device; weights [in, out]."""

    def __init__(self, rt, W, b=None, activation=0):
        super().__init__(rt)
        self.n_in, self.n_out = W.shape
        dW = rt.array(W)
        db = rt.array(b) if b is not None else None
        call("forge_net_linear_create", rt.handle, dW.slice, self.n_in, self.n_out, _sl(db),
             activation, byref(self.h))
        dW.recycle()
        if db is not None:
            db.recycle()

    def _describe(self):
        self.n_in, self.n_out = self._dims()

    def forward(self, X, R=None, pre_out=None, Y=None):
        rows = X.shape[0]
        Y = Y or self.rt.empty((rows, self.n_out))
        call("forge_net_linear_forward", self.h, X.slice, rows, _sl(R), Y.slice, _sl(pre_out))
        return Y

    def backward(self, pre, dY, G, db=None):
        call("forge_net_linear_backward", self.h, _sl(pre), dY.slice, dY.shape[0], G.slice,
             _sl(db))

    def input_gradient(self, G, dX):
        call("forge_net_linear_input_gradient", self.h, G.slice, G.shape[0], dX.slice)

    def learn(self, X, G, db, lr):
        call("forge_net_linear_learn", self.h, X.slice, G.slice, _sl(db), X.shape[0], lr)

    def param(self, which):
        sl = Slice()
        call("forge_net_linear_param", self.h, which, byref(sl))
        shape = (self.n_in, self.n_out) if which == 0 else (self.n_out,)
        return _read(self.rt, sl, shape) if sl.ptr else None


def loss_rows(rt, O, T, out):
    _declare()
    call("forge_net_linear_loss_rows", rt.handle, O.slice, T.slice, O.shape[0], O.shape[1],
         out.slice)


class Mlp(_Model):
    """InferenceMLP / TrainingMlp (mlp.rs:171-269)."""

    def __init__(self, rt, layers, res_range=None, training=False):
        """layers: [(W [in,out] ndarray, b ndarray or None, activation), ...]"""
        super().__init__(rt)
        n = len(layers)
        self.dims = [layers[0][0].shape[0]] + [w.shape[1] for w, _, _ in layers]
        dev = [(rt.array(w), rt.array(b) if b is not None else None) for w, b, _ in layers]
        dims = (c_size_t * (n + 1))(*self.dims)
        acts = (c_int * n)(*[a for _, _, a in layers])
        ws = (Slice * n)(*[d[0].slice for d in dev])
        bs = (Slice * n)(*[_sl(d[1]) for d in dev])
        rs, re_ = (res_range if res_range else (-1, -1))
        call("forge_net_mlp_create", rt.handle, n, dims, acts, ws, bs, rs, re_, int(training),
             byref(self.h))
        for w, b in dev:
            w.recycle()
            if b is not None:
                b.recycle()

    def _describe(self):
        self.dims = self._dims()

    def forward(self, X):
        Y = self.rt.empty((X.shape[0], self.dims[-1]))
        call("forge_net_mlp_forward", self.h, X.slice, X.shape[0], Y.slice)
        return Y

    def backward(self, dY, lr):
        dX = self.rt.empty((dY.shape[0], self.dims[0]))
        call("forge_net_mlp_backward", self.h, dY.slice, dY.shape[0], lr, dX.slice)
        return dX

    def param(self, layer, which):
        sl = Slice()
        call("forge_net_mlp_param", self.h, layer, which, byref(sl))
        shape = (self.dims[layer], self.dims[layer + 1]) if which == 0 else (self.dims[layer + 1],)
        return _read(self.rt, sl, shape) if sl.ptr else None


class Transformer(_Model):
    """encoder/decoder single-head Post-Norm block (encoder.rs, decoder.rs)."""

    def __init__(self, rt, params: dict, seq, hidden, ffn, out, norm_type=LAYER,
                 kind=ENCODER_INFERENCE, qkv_streams=False, ffn_activation=1):
        super().__init__(rt)
        self.desc = TransformerDesc(seq, hidden, ffn, out, norm_type, kind, int(qkv_streams),
                                    ffn_activation)
        self._set_shapes()
        dev = {k: rt.array(v) for k, v in params.items() if v is not None}
        slots = (Slice * len(TP_SLOTS))(*[_sl(dev.get(k)) for k in TP_SLOTS])
        call("forge_net_transformer_create", rt.handle, byref(self.desc), slots, byref(self.h))
        for d in dev.values():
            d.recycle()

    def _set_shapes(self):
        seq, hidden, ffn, out = self.desc.seq, self.desc.hidden, self.desc.ffn, self.desc.out
        self.shapes = {"WQ": (hidden, hidden), "BQ": (hidden,), "WK": (hidden, hidden),
                       "BK": (hidden,), "WV": (hidden, hidden), "BV": (hidden,),
                       "POS": (seq, hidden), "W1": (hidden, ffn), "B1": (ffn,),
                       "W2": (ffn, hidden), "B2": (hidden,), "WO": (hidden, out), "BO": (out,),
                       "G1": (hidden,), "BE1": (hidden,), "G2": (hidden,), "BE2": (hidden,)}

    def _describe(self):
        self.desc = TransformerDesc()
        call("forge_net_transformer_describe", self.h, byref(self.desc))
        self._set_shapes()

    def forward(self, X, Y=None):
        Y = Y or self.rt.empty((self.desc.seq, self.desc.out))
        call("forge_net_transformer_forward", self.h, X.slice, Y.slice)
        return Y

    def backward(self, dY, lr, dX=None, want_grads=False):
        grads = None
        gptr = None
        if want_grads:
            grads = {k: self.rt.empty(self.shapes[k]) for k in TP_SLOTS}
            gptr = (Slice * len(TP_SLOTS))(*[grads[k].slice for k in TP_SLOTS])
        call("forge_net_transformer_backward", self.h, dY.slice, lr, _sl(dX), gptr)
        return grads

    def set_score_bytes(self, nbytes):
        """Largest [seq, seq] score matrix held at once; above it attention
        runs in chunks of query rows (Attention::set_max_score_bytes)."""
        call("forge_net_transformer_set_score_bytes", self.h, nbytes)

    def set_fold_norms(self, on):
        """Inference kinds: fold the parameterless RMSNorms into the
        neighbouring products (on, the default) or run the reference's
        launch order (InferenceBlock::set_fold_norms)."""
        call("forge_net_transformer_set_fold_norms", self.h, 1 if on else 0)

    def param(self, name):
        sl = Slice()
        call("forge_net_transformer_param", self.h, TP_SLOTS.index(name), byref(sl))
        return _read(self.rt, sl, self.shapes[name]) if sl.ptr else None


_KIND_CLASS = {CK_LINEAR: Linear, CK_MLP_INFERENCE: Mlp, CK_MLP_TRAINING: Mlp,
               CK_ENCODER_INFERENCE: Transformer, CK_ENCODER_TRAINING: Transformer,
               CK_DECODER_INFERENCE: Transformer}


def load(rt, path, kind):
    """load_* (model.rs:73-207): a new model of `kind` (a CK_* constant) from
    <path>.toml and its data file."""
    _declare()
    if kind not in _KIND_CLASS:
        raise ValueError(f"unknown checkpoint kind {kind}")
    h = c_void_p()
    call("forge_net_checkpoint_load", rt.handle, os.fsencode(path), kind, byref(h))
    model = _KIND_CLASS[kind].__new__(_KIND_CLASS[kind])
    _Model.__init__(model, rt)
    model.h = h
    model._describe()
    return model


def inspect(path):
    """Validates a checkpoint without a device: (model_type, data_bytes)."""
    _declare()
    buf = ctypes.create_string_buffer(16)
    n = c_uint64()
    call("forge_checkpoint_inspect", os.fsencode(path), buf, len(buf), byref(n))
    return buf.value.decode(), int(n.value)
