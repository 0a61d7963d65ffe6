"""One GDN layer's kernel path after the input projections: conv -> scan ->
gated readout (+ the out_proj input quantization).

Mirrors the kernel branches of ``GatedDeltaNet`` (braid/model/gdn.py): the
decode step ``_decode_kernels`` (:107-167) and the raw-gates chunk prefill
(:273-291), each followed by ``_readout`` (:373-387). The projections
themselves (``project``, :254-255) are GEMMs outside this path, so a layer
here starts from their outputs: ``qkv_proj`` [B, T, C], ``z`` [B, T, H*HD]
(both in the activation dtype) and ``a_raw`` / ``b_raw`` [B, T, H].

Differences from the reference's glue, each a consequence of kernels this
build has and the reference had not:

* prefill's causal conv runs ``conv1d_prefill`` (one launch, window saved in
  place) instead of ``F.conv1d`` over ``[window | x]`` plus a gather
  (gdn.py:193-222); outputs and windows equal ``conv1d_decode`` token by token;
* decode runs the conv and the recurrence as one launch
  (``gdn_conv_decode_raw``) where the shape allows, instead of
  ``conv1d_decode`` then ``gdn_decode_raw`` (gdn.py:131-160), same bits;
* the readout runs ``gated_rmsnorm`` (norm, gate and, for an FP8 out_proj,
  the activation quantization in two launches) instead of the torch norm and
  ``quantize_act``.

The return value is what ``out_proj`` consumes: ``(core, xq, sx)`` when the
out_proj weight is FP8 (``fp8_out``), else ``core``.
"""
from __future__ import annotations

from typing import Optional

import torch

from braid_amd.cache import RecurrentCache
from braid_amd.config import GDNConfig
from braid_amd.kernels.loader import load_gdn


class GDNMixerLayer:
    """Weights as the reference holds them after loading (gdn.py:83-97,
    braid/model/loader.py:185-195): ``conv1d`` [C, K] (any float dtype, kept
    as an fp32 copy), ``conv1d_bias`` [C] or absent, ``A`` [H] fp32
    (= -exp(A_log)), ``dt_bias`` [H] fp32, ``norm`` [HD] fp32 (gamma stored
    directly, no unit offset)."""

    def __init__(self, g: GDNConfig, weights: dict, eps: float = 1e-6, fp8_out: bool = True):
        self.g = g
        self.eps = float(eps)
        self.fp8_out = fp8_out
        # fp32 copies made once: a cast allocates, and an allocation inside a
        # captured graph is a capture failure (gdn.py:89-95).
        self.conv1d_f32 = weights["conv1d"].float().contiguous()
        bias = weights.get("conv1d_bias")
        self.conv_bias_f32 = None if bias is None else bias.float().contiguous()
        self.A = weights["A"].float().contiguous()
        self.dt_bias = weights["dt_bias"].float().contiguous()
        self.norm = weights["norm"].float().contiguous()
        self._mod = load_gdn()
        # The fused conv + recurrence launch covers conv kernel 4 with one or
        # two value heads per key group (every Qwen3.5 GDN layer); other shapes
        # run the two kernels. Either way the bits are the same.
        self.fused_decode = (g.conv_kernel == 4 and g.n_heads // g.n_groups in (1, 2))

    def _split(self, conv_out: torch.Tensor):
        """[..., C] -> q, k [..., G, SS] and v [..., H, HD]; Q | K | V, Q first
        (braid/config.py:34-44). Views, not copies (gdn.py:143-156)."""
        g = self.g
        q, k, v = torch.split(conv_out, [g.key_dim, g.key_dim, g.inner_size], dim=-1)
        return (q.unflatten(-1, (g.n_groups, g.state_size)),
                k.unflatten(-1, (g.n_groups, g.state_size)),
                v.unflatten(-1, (g.n_heads, g.head_dim)))

    def _readout(self, z: torch.Tensor, y: torch.Tensor):
        return self._mod.gated_rmsnorm(y, z.contiguous(), self.norm, self.eps,
                                       quantize=self.fp8_out)

    def decode(self, qkv_proj: torch.Tensor, z: torch.Tensor, a_raw: torch.Tensor,
               b_raw: torch.Tensor, cache: RecurrentCache, slots_i32: torch.Tensor):
        """One token for every row: qkv_proj [B, 1, C], z [B, 1, H*HD],
        a_raw / b_raw [B, 1, H] (gdn.py:107-167 with raw gates, then _readout).
        The conv and the recurrence run as one fused launch when the shape
        allows it (conv kernel 4, one or two value heads per key group), with
        the same bits as the two kernels back to back."""
        g = self.g
        B = qkv_proj.shape[0]
        qkv = qkv_proj[:, 0]
        y = torch.empty(B, 1, g.n_heads, g.head_dim, device=qkv.device, dtype=torch.float32)
        if self.fused_decode:
            self._mod.gdn_conv_decode_raw(cache.state, cache.conv, slots_i32, qkv.contiguous(),
                                          self.conv1d_f32, self.conv_bias_f32,
                                          a_raw[:, 0].contiguous(), b_raw[:, 0].contiguous(),
                                          self.A, self.dt_bias, y[:, 0], g.n_groups)
            return self._readout(z, y)
        conv_out = torch.empty(qkv.shape, device=qkv.device, dtype=torch.float32)
        self._mod.conv1d_decode(cache.conv, slots_i32, qkv.contiguous(), self.conv1d_f32,
                                self.conv_bias_f32, conv_out)
        q, k, v = self._split(conv_out)
        self._mod.gdn_decode_raw(cache.state, slots_i32, q, k, v, a_raw[:, 0].contiguous(),
                                 b_raw[:, 0].contiguous(), self.A, self.dt_bias, y[:, 0])
        return self._readout(z, y)

    def prefill(self, qkv_proj: torch.Tensor, z: torch.Tensor, a_raw: torch.Tensor,
                b_raw: torch.Tensor, cache: RecurrentCache, slots_i32: torch.Tensor,
                seq_lens: Optional[torch.Tensor] = None, plan_lens: Optional[list] = None):
        """T tokens per row, right-padded when ``seq_lens`` is given (row b owns
        columns 0..seq_lens[b]-1): conv prefill, raw-gates chunk scan, readout
        (gdn.py:171-226 and :273-291). Pad columns leave the conv window and the
        state exactly as the row's last live token left them. ``plan_lens``: the
        same lengths on the host, for a captured call to plan its ragged scan
        from (``gdn_prefill_raw``); the bits do not depend on it."""
        g = self.g
        if cache is None or slots_i32 is None:
            raise ValueError("a pooled cache needs a slot assignment")
        B, T, C = qkv_proj.shape
        lens = None if seq_lens is None else seq_lens.to(torch.int32).contiguous()
        conv_out = torch.empty(B, T, C, device=qkv_proj.device, dtype=torch.float32)
        self._mod.conv1d_prefill(cache.conv, slots_i32, qkv_proj.contiguous(), self.conv1d_f32,
                                 self.conv_bias_f32, conv_out, lens)
        q, k, v = self._split(conv_out)
        y = torch.empty(B, T, g.n_heads, g.head_dim, device=qkv_proj.device,
                        dtype=torch.float32)
        self._mod.gdn_prefill_raw(cache.state, slots_i32, q.contiguous(), k.contiguous(),
                                  v.contiguous(), a_raw.contiguous(), b_raw.contiguous(),
                                  self.A, self.dt_bias, y, lens,
                                  plan_lens=plan_lens if lens is not None else None)
        return self._readout(z, y)


def mixer_decode_step(layers: list):
    """A decode step over a stack of layers, in the form ``GraphedDecoder``
    captures: ``step(inputs, view)`` with ``inputs`` holding per-layer lists
    ``qkv``, ``z``, ``a``, ``b`` of [B, 1, ...] tensors and ``view`` a
    ``GDNCache`` whose ``slots_i32`` names the rows' slots. Returns the
    per-layer readouts."""

    def step(inputs: dict, view) -> list:
        return [lyr.decode(inputs["qkv"][i], inputs["z"][i], inputs["a"][i], inputs["b"][i],
                           view.layers[i], view.slots_i32)
                for i, lyr in enumerate(layers)]

    return step
