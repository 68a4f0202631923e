"""VQ MoE block for PyTorch-ROCm: SwitchGLU + SparseMoeBlock over VQ experts.

The reference serves MoE layers through mlx-lm's SwitchGLU and
SparseMoeBlock with VQSwitchLinear projections swapped in
(bundle/add_model_file.py:70-131); its routing and combine are restated in
bench/decode_ladder.py:107-119 and tests/test_qwen3_5_parity.py:180-205:

    probs = softmax(logits) (fp32); ids = top_k(probs); w = probs[ids]
    w /= w.sum() (norm_topk_prob)
    y = sum_j w_j * down_j(silu(gate_j(x)) * up_j(x))
        + sigmoid(shared_expert_gate(x)) * shared_expert(x)

VQSparseMoeBlock runs that whole block as one fused decode layer
(vqk_moe_decode_layer: routing on device, one or two kernels, no host sync)
when the shapes fit, and otherwise composes the per-projection kernels
(VQSwitchLinear) with torch's routing ops on the same device.
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import _lib as L
from . import _torch as T
from .vq_switch import VQSwitchLinear


class VQSwitchGLU(torch.nn.Module):
    """mlx-lm SwitchGLU with VQ projections: down(silu(gate(x)) * up(x)) per
    routed expert. x [..., H], indices [..., k] -> [..., k, H]. gate/up leave
    in fp32 and the SwiGLU product enters down_proj as fp16, the numerics of
    the fused layer (mlx-lm rounds both to the activation dtype)."""

    def __init__(self, gate_proj: VQSwitchLinear, up_proj: VQSwitchLinear,
                 down_proj: VQSwitchLinear):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def forward(self, x, indices, out_dtype=None):
        xe = x[..., None, None, :]
        g = self.gate_proj(xe, indices, out_dtype=torch.float32)
        u = self.up_proj(xe, indices, out_dtype=torch.float32)
        h = (F.silu(g) * u).to(torch.float16)                        # [..., k, 1, I]
        y = self.down_proj(h, indices, out_dtype=out_dtype or x.dtype)   # [..., k, 1, H]
        return y.squeeze(-2)


def _desc_of(mod: VQSwitchLinear, keep):
    return T.weights(mod.codes, mod.codebook, mod.vq_scales, mod.group_size, mod.pack_bits,
                     mod.input_dims, mod.row_table, k_expect=mod._k_expect, keep=keep)


class VQSparseMoeBlock(torch.nn.Module):
    """Routed VQ experts + optional shared expert, as one decode layer.

    switch_mlp: VQSwitchGLU over E experts; shared_expert: VQSwitchGLU over
    one expert (E == 1) or None; shared_expert_gate: [H] weights of the
    shared gate linear. forward(x [T, H], logits [T, E]) -> [T, H].
    """

    def __init__(self, switch_mlp: VQSwitchGLU, top_k: int, norm_topk_prob: bool = True,
                 shared_expert: VQSwitchGLU | None = None, shared_expert_gate=None,
                 router_weight=None):
        super().__init__()
        self.switch_mlp = switch_mlp
        self.top_k = int(top_k)
        self.norm_topk_prob = bool(norm_topk_prob)
        self.shared_expert = shared_expert
        self.shared_expert_gate = shared_expert_gate
        self.router_weight = router_weight
        self._ws = None

    @classmethod
    def from_modules(cls, projs, top_k, in_features, shared=None, shared_gate=None,
                     norm_topk_prob=True):
        """projs: {"gate"|"up"|"down": (codes, codebook, scales, pack_bits)}."""
        def lin(spec, name):
            codes, cb, sc, pb = spec
            return VQSwitchLinear(codes, cb, sc, pack_bits=pb,
                                  in_features=in_features[name] if pb else None)
        mlp = VQSwitchGLU(lin(projs["gate"], "gate"), lin(projs["up"], "up"),
                          lin(projs["down"], "down"))
        sh = None
        if shared is not None:
            sh = VQSwitchGLU(lin(shared["gate"], "gate"), lin(shared["up"], "up"),
                             lin(shared["down"], "down"))
        return cls(mlp, top_k, norm_topk_prob, sh, shared_gate)

    # -------------------------------------------------------------- fused
    def _fused_desc(self, keep):
        m = self.switch_mlp
        d = L.VQKMoeDesc()
        ws = [_desc_of(m.gate_proj, keep), _desc_of(m.up_proj, keep), _desc_of(m.down_proj, keep)]
        keep.extend(ws)
        d.gate, d.up, d.down = (ctypes.pointer(w) for w in ws)
        if self.shared_expert is not None:
            s = self.shared_expert
            sw = [_desc_of(s.gate_proj, keep), _desc_of(s.up_proj, keep),
                  _desc_of(s.down_proj, keep)]
            keep.extend(sw)
            d.sh_gate, d.sh_up, d.sh_down = (ctypes.pointer(w) for w in sw)
            g = self.shared_expert_gate.reshape(-1).contiguous()
            keep.append(g)
            d.sh_gate_vec = g.data_ptr()
            d.sh_gate_vec_type = T.act_type(g)
        d.top_k = self.top_k
        d.norm_topk = int(self.norm_topk_prob)
        return d

    def fused(self, x, logits, return_route=False):
        """One fused decode layer; raises NotImplementedError for shapes the
        fused kernels do not cover."""
        T.require_cuda(x, logits)
        keep = []
        d = self._fused_desc(keep)
        Tt = x.shape[0]
        x = x.contiguous()
        lg = logits.float().contiguous()
        ws = ctypes.c_size_t()
        L.check(L.lib().vqk_moe_decode_layer_workspace(ctypes.byref(d), Tt, ctypes.byref(ws)),
                "moe layer")
        if self._ws is None or self._ws.numel() < ws.value or self._ws.device != x.device:
            # the header (call number, error word, hand-off words) starts zeroed
            self._ws = torch.zeros(max(ws.value, L.VQK_MOE_HEADER_BYTES), dtype=torch.uint8,
                                   device=x.device)
        y = torch.empty((Tt, x.shape[1]), dtype=x.dtype, device=x.device)
        ids = torch.empty((Tt, self.top_k), dtype=torch.int32, device=x.device) if return_route else None
        w = torch.empty((Tt, self.top_k), dtype=torch.float32, device=x.device) if return_route else None
        L.check(L.lib().vqk_moe_decode_layer(ctypes.byref(d), T.ptr(x), T.act_type(x), Tt,
                                             T.ptr(lg), T.ptr(y), T.act_type(y), T.ptr(ids),
                                             T.ptr(w), T.ptr(self._ws), ws.value,
                                             T.stream(x.device)), "moe layer")
        return (y, ids, w) if return_route else y

    def status(self):
        """Raise RuntimeError if a one-launch call on this block's workspace
        gave up a wait (its rows, and those of every later one-launch call
        until reset(), are NaN); synchronises the current stream."""
        if self._ws is not None:
            L.check(L.lib().vqk_moe_layer_status(T.ptr(self._ws), T.stream(self._ws.device)),
                    "moe layer")

    def reset(self):
        """Zero the workspace header (clears a reported error)."""
        if self._ws is not None:
            L.check(L.lib().vqk_moe_layer_reset(T.ptr(self._ws), T.stream(self._ws.device)),
                    "moe layer")

    # ----------------------------------------------------------- composed
    def composed(self, x, logits):
        probs = torch.softmax(logits.float(), dim=-1)
        w, ids = torch.topk(probs, self.top_k, dim=-1, sorted=True)
        if self.norm_topk_prob:
            w = w / w.sum(-1, keepdim=True)
        ye = self.switch_mlp(x, ids.to(torch.int32), out_dtype=torch.float32)   # [T, k, H]
        y = (ye * w[..., None]).sum(-2)
        if self.shared_expert is not None:
            sid = torch.zeros((x.shape[0], 1), dtype=torch.int32, device=x.device)
            sy = self.shared_expert(x, sid, out_dtype=torch.float32)[:, 0]
            sg = torch.sigmoid(x.float() @ self.shared_expert_gate.reshape(-1).float())
            y = y + sg[:, None] * sy
        return y.to(x.dtype)

    def forward(self, x, logits=None):
        if logits is None:
            logits = x.float() @ self.router_weight.float().T
        try:
            return self.fused(x, logits)
        except NotImplementedError:
            return self.composed(x, logits)
