"""LUT transformer: token embedding -> [LUT attention (sequence-concat LUT
layer) + residual -> LUT feed-forward + residual] x num_layers -> LUT
unembedding (reference src/spiky/lut/LUTTransformer.py:15-480).

Every LUT layer runs on this build's HIP kernels: the attention layers are
`LUTLayer`s with `sequence_length = context_size` (causal pairs i < j, rows
Q_j | K_i | PE_(j-i-1)); the feed-forward and unembedding layers are
`LUTLayer`s applied to the [B*S, 1, E] reshape of the activations.  A 2-D
`embedding_dim` (h, w) makes each attention layer a `Conv2DLUTLayer` over the
[h, w] grid with one receptive field covering it (sparse lookup connectivity,
LUTTransformer.py:43-67); everything else sees E = h * w features.
"""
import torch
import torch.nn as nn

from .LUTLayer import Conv2DLUTLayer, GradientPolicy, LUTLayer, LUTSharedContext, SynapseMeta


class LUTTransformer(nn.Module):
    """Constructor arguments and seeding follow the reference
    (LUTTransformer.py:69-200): attention layer l is seeded seed + l*num_heads,
    its feed-forward layer seed + l*num_heads + num_heads, the unembedder seed;
    the frozen embedding is 2*U[0,1) - 1 from a generator seeded with seed
    (else uniform(-1, 1) from the global RNG)."""

    def __init__(self, vocab_size, embedding_dim, context_size, positional_dim, num_layers, num_heads,
                 n_detectors, n_anchors_per_detector, n_anchors_per_detector_attention=None,
                 no_ffn=False, concatenation_product=True, sliced_product_mode=False, unified_pe=False,
                 do_normalise_weights=False, weights_gradient_policy: GradientPolicy = None,
                 device=None, synapse_meta=SynapseMeta(), lut_shared_context=None, seed=None,
                 summation_dtype=torch.float32, _int_rescaler=0.001, _forward_group_size=32,
                 _backward_group_size=32, dropout=0.0, use_batch_norm=False):
        super().__init__()
        if isinstance(embedding_dim, int):
            n_embeddings = embedding_dim
        else:
            # LUTTransformer.py:111-115
            embedding_dim = tuple(embedding_dim)
            assert len(embedding_dim) == 2
            n_embeddings = embedding_dim[0] * embedding_dim[1]
        self.vocab_size = vocab_size
        self.embedding_dim = embedding_dim
        self.context_size = context_size
        self.positional_dim = positional_dim
        self.num_layers = num_layers
        self.num_heads = num_heads
        self.n_detectors = n_detectors
        self.n_anchors_per_detector = n_anchors_per_detector
        self.n_anchors_per_detector_attention = (n_anchors_per_detector_attention
                                                 if n_anchors_per_detector_attention is not None
                                                 else n_anchors_per_detector)
        self.concatenation_product = concatenation_product
        self.sliced_product_mode = sliced_product_mode
        self.weights_gradient_policy = weights_gradient_policy
        self.dropout = dropout
        self.use_batch_norm = use_batch_norm
        self.unified_pe = unified_pe
        self.no_ffn = no_ffn
        self.device = torch.device("cpu") if device is None else torch.device(device)
        if lut_shared_context is None:
            lut_shared_context = LUTSharedContext()
            lut_shared_context.to_device(self.device)
        self.lut_shared_context = lut_shared_context

        E = n_embeddings
        self.token_embedder = nn.Embedding(vocab_size, E, device=self.device)
        self.token_embedder.weight.requires_grad_(False)
        with torch.no_grad():
            if seed is not None:
                gen = torch.Generator(device=self.device)
                gen.manual_seed(seed)
                self.token_embedder.weight.copy_(
                    2 * torch.rand(self.token_embedder.weight.shape, generator=gen, device=self.device) - 1.0)
            else:
                nn.init.uniform_(self.token_embedder.weight, -1.0, 1.0)

        common = dict(synapse_meta=synapse_meta, do_normalise_weights=do_normalise_weights,
                      weights_gradient_policy=weights_gradient_policy, shared_context=self.lut_shared_context,
                      summation_dtype=summation_dtype, _int_rescaler=_int_rescaler, device=self.device,
                      _forward_group_size=_forward_group_size, _backward_group_size=_backward_group_size)
        self.layers = nn.ModuleList()
        for li in range(num_layers):
            block = nn.ModuleDict()
            attention_seed = None if seed is None else seed + li * num_heads
            if isinstance(embedding_dim, int):
                block["attention_lut"] = LUTLayer(
                    n_inputs=E, n_anchors_per_detector=self.n_anchors_per_detector_attention,
                    n_detectors=n_detectors * num_heads, n_outputs=E, sequence_length=context_size,
                    concatenation_product=concatenation_product, sliced_product_mode=sliced_product_mode,
                    positional_dim=positional_dim, unified_pe=unified_pe, random_seed=attention_seed,
                    **common)
            else:
                # LUTTransformer.py:43-67
                block["attention_lut"] = Conv2DLUTLayer(
                    input_shape=embedding_dim, n_anchors_per_detector=self.n_anchors_per_detector_attention,
                    detectors_shape=(1, n_detectors * num_heads), output_kernel_shape=embedding_dim,
                    sequence_length=context_size, concatenation_product=concatenation_product,
                    sliced_product_mode=sliced_product_mode, positional_dim=positional_dim,
                    unified_pe=unified_pe, receptive_field_shape=embedding_dim,
                    receptive_field_stride_shape=embedding_dim, random_seed=attention_seed, **common)
            block["attention_dropout"] = nn.Dropout(dropout)
            block["attention_bn"] = nn.BatchNorm1d(E, device=self.device) if use_batch_norm else None
            if not no_ffn:
                block["ffn"] = LUTLayer(
                    n_inputs=E, n_anchors_per_detector=n_anchors_per_detector, n_detectors=n_detectors,
                    n_outputs=E, sequence_length=1,
                    random_seed=None if seed is None else seed + li * num_heads + num_heads, **common)
                block["ffn_dropout"] = nn.Dropout(dropout)
                block["ffn_bn"] = nn.BatchNorm1d(E, device=self.device) if use_batch_norm else None
            self.layers.append(block)
        self.unembedder = LUTLayer(n_inputs=E, n_anchors_per_detector=n_anchors_per_detector,
                                   n_detectors=n_detectors, n_outputs=vocab_size, sequence_length=1,
                                   random_seed=seed, **common)
        self._debug_last_forward = None

    def _lut_layers(self):
        for block in self.layers:
            yield block["attention_lut"]
            if not self.no_ffn:
                yield block["ffn"]
        yield self.unembedder

    def set_external_learning_rate_hook(self, lr_hook):
        for layer in self._lut_layers():
            layer.set_external_learning_rate_hook(lr_hook)

    def _reset_shared_context(self, new_context):
        for layer in self._lut_layers():
            layer._reset_shared_context(new_context)

    @staticmethod
    def _bn(bn, z):
        # BatchNorm1d over the embedding features of every (sample, position)
        return bn(z.reshape(-1, z.shape[-1])).reshape(z.shape)

    def forward(self, tokens):
        """tokens [B, S] -> logits [B, S, vocab_size] (LUTTransformer.py:209-271)."""
        B, S = tokens.shape[0], self.context_size
        grid = not isinstance(self.embedding_dim, int)
        E = self.embedding_dim[0] * self.embedding_dim[1] if grid else self.embedding_dim
        z = self.token_embedder(tokens)
        if self._debug_last_forward is not None:
            self._debug_last_forward = [tokens.to(torch.float32), z.detach().clone()]
        for block in self.layers:
            if grid:
                z = z.reshape((B, S) + self.embedding_dim)
            a = block["attention_lut"](z)
            if self._debug_last_forward is not None:
                self._debug_last_forward.append(a.detach().clone())
            a = block["attention_dropout"](a)
            if self.use_batch_norm:
                a = self._bn(block["attention_bn"], a)
            z = z + a
            if grid:
                z = z.reshape(B, S, E)
            if not self.no_ffn:
                f = block["ffn"](z.reshape(B * S, 1, E)).reshape(B, S, E)
                if self._debug_last_forward is not None:
                    self._debug_last_forward.append(f.detach().clone())
                f = block["ffn_dropout"](f)
                if self.use_batch_norm:
                    f = self._bn(block["ffn_bn"], f)
                z = z + f
        return self.unembedder(z.reshape(B * S, 1, E)).reshape(B, S, self.vocab_size)

    def to(self, *args, **kwargs):
        device = kwargs.get("device", args[0] if args and isinstance(args[0], (str, torch.device)) else None)
        if device is not None:
            dev = torch.device(device)
            if dev.type == "cuda" and dev.index is None:
                dev = torch.device("cuda", torch.cuda.current_device())
            self.device = dev
            self.lut_shared_context.to_device(dev)
        super().to(*args, **kwargs)
        for layer in self._lut_layers():
            if device is not None:
                layer.to(device=self.device)
        return self

    def get_profile_statistics(self) -> str:
        """Per-layer profiler output of every LUT layer (LUTTransformer.py:345-480)."""
        lines = []
        for i, block in enumerate(self.layers):
            lines.append(f"layer {i} attention:\n{block['attention_lut'].get_profiling_stats()}")
            if not self.no_ffn:
                lines.append(f"layer {i} ffn:\n{block['ffn'].get_profiling_stats()}")
        lines.append(f"unembedder:\n{self.unembedder.get_profiling_stats()}")
        return "\n".join(lines)
