"""A small attention-only language model for executor tests (test infrastructure).

Every layer projects the hidden states to Q/K/V, rotates Q and K by their
absolute positions (rotate-half RoPE, base 10000), hands attention to the
backend it is given -- the TPRAttentionBackend seam of attention.py:141-148 --
and adds the projected output back. The loss is a summed cross entropy
against deterministic targets. ``forward_fn`` has the signature the
executor calls; ``dense_path_loss`` runs the same model on one segment's whole
root path with ordinary causal attention (the oracle's, on the CPU)."""

from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle.tpr_oracle import prefix_attention


class ToyModel:
    def __init__(self, *, vocab=64, hidden=256, hq=8, hkv=2, d=128, layers=2, seed=0, dtype=torch.float64,
                 device="cpu", params=None):
        self.vocab, self.hidden, self.hq, self.hkv, self.d, self.layers = vocab, hidden, hq, hkv, d, layers
        self.dtype, self.device = dtype, torch.device(device)
        if params is None:
            gen = torch.Generator(device="cpu").manual_seed(seed)

            def w(*shape, fan_in):
                return torch.randn(*shape, generator=gen) / fan_in ** 0.5

            params = {"emb": w(vocab, hidden, fan_in=1), "out": w(hidden, vocab, fan_in=hidden)}
            for layer in range(1, layers + 1):
                params[f"wq{layer}"] = w(hidden, hq * d, fan_in=hidden)
                params[f"wk{layer}"] = w(hidden, hkv * d, fan_in=hidden)
                params[f"wv{layer}"] = w(hidden, hkv * d, fan_in=hidden)
                params[f"wo{layer}"] = w(hq * d, hidden, fan_in=hq * d)
        self.params = {n: p.detach().to(dtype).to(self.device).requires_grad_(True) for n, p in params.items()}

    def clone_to(self, dtype, device):
        """The same weights (values as stored here) in another dtype / device."""
        return ToyModel(vocab=self.vocab, hidden=self.hidden, hq=self.hq, hkv=self.hkv, d=self.d,
                        layers=self.layers, dtype=dtype, device=device,
                        params={n: p.detach().cpu() for n, p in self.params.items()})

    def grads(self):
        return {n: (p.grad.detach().clone() if p.grad is not None else torch.zeros_like(p)) for n, p in
                self.params.items()}

    # -- pieces ---------------------------------------------------------------------
    def _rope(self, x, positions):
        half = self.d // 2
        inv = 1.0 / (10000.0 ** (torch.arange(0, half, device=x.device, dtype=torch.float64) / half))
        ang = positions.to(torch.float64)[:, None] * inv[None, :]
        cos = ang.cos()[:, None, None, :]
        sin = ang.sin()[:, None, None, :]
        cdt = torch.float64 if x.dtype == torch.float64 else torch.float32
        xf = x.to(cdt)
        x1, x2 = xf[..., :half], xf[..., half:]
        cos, sin = cos.to(cdt), sin.to(cdt)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1).to(x.dtype)

    @staticmethod
    def targets(ids, vocab):
        return (ids * 7 + 3) % vocab

    def _run(self, ids, positions, attend):
        p = self.params
        h = p["emb"][ids]
        n = ids.shape[0]
        new_kv = {}
        for layer in range(1, self.layers + 1):
            q = (h @ p[f"wq{layer}"]).view(n, 1, self.hq, self.d)
            k = (h @ p[f"wk{layer}"]).view(n, 1, self.hkv, self.d)
            v = (h @ p[f"wv{layer}"]).view(n, 1, self.hkv, self.d)
            q, k = self._rope(q, positions), self._rope(k, positions)
            o = attend(layer, q, k, v)                       # [n, 1, hq * d]
            h = h + o[:, 0] @ p[f"wo{layer}"]
            new_kv[layer] = (k, v)
        logits = h @ p["out"]
        if logits.dtype not in (torch.float32, torch.float64):
            logits = logits.float()
        return logits, new_kv

    # -- the executor's forward ---------------------------------------------------------
    def forward_fn(self, tokens):
        """tokens: {segment_id: LongTensor [length]}."""

        def run(segs, positions, backend):
            ids = torch.cat([tokens[s.segment_id] for s in segs]).to(self.device)
            logits, new_kv = self._run(ids, positions.to(self.device),
                                       lambda layer, q, k, v: backend.attention(layer, q, k, v, softmax_scale=None))
            loss = F.cross_entropy(logits, self.targets(ids, self.vocab), reduction="sum")
            return loss, new_kv

        return run

    def dense_path_loss(self, path_tokens, own_length):
        """The loss of the last ``own_length`` tokens of ``path_tokens`` (a root
        path, positions 0..), computed with one dense causal attention over the
        whole path (prefix length 0)."""
        ids = path_tokens.to(self.device)
        positions = torch.arange(ids.shape[0], device=self.device)

        def attend(layer, q, k, v):
            empty = k[:0]
            return prefix_attention(q, k, v, empty, empty, None)

        logits, _ = self._run(ids, positions, attend)
        own = slice(ids.shape[0] - own_length, ids.shape[0])
        return F.cross_entropy(logits[own], self.targets(ids[own], self.vocab), reduction="sum")
