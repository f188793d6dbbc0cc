"""GenerativeSnapshot and ActivationType, mirroring the reference's model handoff.

GenerativeSnapshot (Networks/GenerativeSnapshot.cs:15-23): LayerSizes, the
activation, StateLearningRate (eta), ActivityRegularization (lambda),
UseFeedforwardGistInit, Weights[l-1] = W_l [s_{l-1} x s_l], Biases[l-1] = b_l
[s_{l-1}] and one scalar precision per layer.  Like
Network.ExportGenerativeSnapshot (Network.cs:1328-1356) it refuses per-unit
(diagonal) precisions and prior means, which the batched relaxation does not
reproduce.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import IntEnum

import numpy as np

from .errors import ArgumentException, NotSupportedException


class ActivationType(IntEnum):
    """Activation.cs:19-25, extended with the tanh-approximation GELU
    (PredictiveCoding.LLM/Model/Layers.cs:42-50)."""
    Linear = 0
    Tanh = 1
    ReLU = 2
    Sigmoid = 3
    Gelu = 4


@dataclass
class GenerativeSnapshot:
    layer_sizes: list
    activation: ActivationType
    state_learning_rate: float
    activity_regularization: float
    use_feedforward_gist_init: bool
    weights: list
    biases: list
    precisions: list = field(default=None)
    prior_mean: object = None

    def __post_init__(self):
        L = len(self.layer_sizes)
        if L < 2:
            raise ArgumentException("a generative model needs at least two layers")
        self.layer_sizes = [int(s) for s in self.layer_sizes]
        self.activation = ActivationType(self.activation)
        if self.precisions is None:
            self.precisions = [1.0] * L
        if len(self.weights) != L - 1 or len(self.biases) != L - 1 or len(self.precisions) != L:
            raise ArgumentException("weights/biases/precisions do not match the layer count")
        if self.prior_mean is not None:
            raise NotSupportedException(
                "GenerativeSnapshot does not support informative priors -- "
                "the batched forward would not reproduce the network's dynamics.")
        for p in self.precisions:
            if np.ndim(p) != 0:
                raise NotSupportedException(
                    "GenerativeSnapshot does not support diagonal precision -- "
                    "the batched forward would not reproduce the network's dynamics.")
        ws, bs = [], []
        for l in range(1, L):
            # Own copies, read-only: the snapshot is immutable once made.  The
            # drop-in uploads a snapshot's weights once and reuses the device
            # copy on later calls, where the reference re-reads model.Weights
            # on every call (BatchedPcForward.cs:62-64); an edit of the caller's
            # arrays after construction therefore must not reach the snapshot,
            # and an edit through the snapshot is refused (ValueError).
            w = np.array(self.weights[l - 1], dtype=np.float32, order="C", copy=True)
            b = np.array(self.biases[l - 1], dtype=np.float32, copy=True).ravel()
            if w.shape != (self.layer_sizes[l - 1], self.layer_sizes[l]):
                raise ArgumentException(f"W_{l} has shape {w.shape}, expected "
                                        f"({self.layer_sizes[l - 1]}, {self.layer_sizes[l]})")
            if b.shape != (self.layer_sizes[l - 1],):
                raise ArgumentException(f"b_{l} has shape {b.shape}, expected ({self.layer_sizes[l - 1]},)")
            w.setflags(write=False)
            b.setflags(write=False)
            ws.append(w)
            bs.append(b)
        self.weights, self.biases = tuple(ws), tuple(bs)
        self.precisions = tuple(float(p) for p in self.precisions)
        self.layer_sizes = tuple(self.layer_sizes)
        object.__setattr__(self, "_frozen", True)

    def __setattr__(self, name, value):
        # Fields are set once, in __init__/__post_init__; a new model is a new
        # snapshot (Network.ExportGenerativeSnapshot makes one per call).
        if getattr(self, "_frozen", False):
            raise NotSupportedException(f"GenerativeSnapshot is immutable: cannot set {name!r}; "
                                        "export a new snapshot instead.")
        object.__setattr__(self, name, value)
