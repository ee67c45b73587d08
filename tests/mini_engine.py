"""A small decode engine for the GPU tests, built from qengine_amd's ops the way the reference's
engine drives qengine._C (python/qengine/engine.py:384-520): per-layer rmsnorm1p with the fused
residual, in_proj GEMV, attn_prep, attn_decode, o_proj GEMV, SwiGLU MLP, final norm, lm_head
GEMV, argmax, accept and commit, all on device buffers, one hipGraph per pass width. Weights are
random (there is no checkpoint here). Layers are gated-attention layers, or Gated DeltaNet layers
(in_proj GEMV, gdn_step_n with its lazy rollback, out_proj GEMV) where ``layer_types`` says
"linear_attention", as in the reference's hybrid model (engine.py:436-448).

Test infrastructure: it exists to check that a whole step runs as one graph and that
speculative verify passes reproduce plain greedy decoding token for token.
"""
from __future__ import annotations

import torch

import qengine_amd as qa

BF, I32, F32 = torch.bfloat16, torch.int32, torch.float32
NMAX = 8
HD = 256


class MiniEngine:
    def __init__(self, layers=2, hidden=1024, inter=2048, vocab=4096, hq=24, hkv=4, max_len=256,
                 seed=0, device="cuda", layer_types=None, hk=4, hv=8):
        self.dev, self.H, self.I, self.V, self.hq, self.hkv = device, hidden, inter, vocab, hq, hkv
        self.types = list(layer_types or ["full_attention"] * layers)
        assert len(self.types) == layers
        self.hk, self.hv = hk, hv
        self.max_len, self.eps = max_len, 1e-6
        g = torch.Generator(device=device).manual_seed(seed)

        def w(n, k, scale=1.0):
            return (torch.randn(n, k, device=device, generator=g) * (scale * k ** -0.5)).to(BF)

        def norm_w(n):
            return (torch.randn(n, device=device, generator=g) * 0.1).to(BF)

        H, I = hidden, inter
        self.attn_n = hq * 2 * HD + 2 * hkv * HD
        self.conv_dim = 2 * hk * 128 + hv * 128
        self.gdn_n = self.conv_dim + hv * 128 + 2 * hv
        self.embed_t = (torch.randn(vocab, H, device=device, generator=g)).to(BF)
        self.layers = []
        for t in self.types:
            L = dict(type=t, in_norm=norm_w(H), post_norm=norm_w(H), gate_up=w(2 * I, H),
                     down=w(H, I))
            if t == "linear_attention":
                L.update(
                    in_proj=w(self.gdn_n, H), out=w(H, hv * 128),
                    conv_w=(torch.randn(self.conv_dim, 1, 4, device=device, generator=g) * 0.5).to(BF),
                    A_log=(torch.rand(hv, device=device, generator=g) * 2 - 1).to(BF),
                    dt_bias=torch.randn(hv, device=device, generator=g).to(BF),
                    norm_w=(1 + 0.1 * torch.randn(128, device=device, generator=g)).to(BF),
                    ring=torch.zeros(16, self.conv_dim, dtype=BF, device=device),
                    S=torch.zeros(hv, 128, 128, device=device),
                    st=[torch.zeros(NMAX, hv, 128, device=device),
                        torch.zeros(NMAX, hv, 128, device=device),
                        torch.zeros(NMAX, hv, 2, device=device)])
            else:
                L.update(q_norm=norm_w(HD), k_norm=norm_w(HD), in_proj=w(self.attn_n, H),
                         out=w(H, hq * HD),
                         kc=torch.zeros(hkv, max_len, HD, dtype=BF, device=device),
                         vc=torch.zeros(hkv, max_len, HD, dtype=BF, device=device))
            self.layers.append(L)
        self.final_norm = norm_w(H)
        self.lm_head = w(vocab, H, scale=4.0)
        z = lambda *s, dt=BF: torch.zeros(*s, dtype=dt, device=device)  # noqa: E731
        self.ctl = z(32, dt=I32)
        self.in_tok = z(NMAX + 1, dt=I32)
        self.am, self.next_tok, self.drafts = z(NMAX, dt=I32), z(NMAX, dt=I32), z(NMAX, dt=I32)
        self.log = z(max_len, dt=I32)
        self.h, self.xn, self.mo, self.hid = z(NMAX, H), z(NMAX, H), z(NMAX, H), z(NMAX, H)
        self.proj = z(NMAX, (max(self.attn_n, self.gdn_n) + 7) // 8 * 8)
        self.mix = z(NMAX, max(hq * HD, hv * 128))
        self.gu, self.act = z(NMAX, 2 * I), z(NMAX, I)
        self.logits = z(NMAX, vocab)
        self.am_v, self.am_i = z(NMAX * 256, dt=F32), z(NMAX * 256, dt=I32)
        self.q = z(NMAX, hq * HD)
        ns = qa.default_splits(max_len, hkv)
        self.part_o, self.part_ml = qa.alloc_partials(NMAX, hq, ns, device)
        self.inv_freq = (1.0 / (1e7 ** (torch.arange(0, 64, 2, dtype=F32) / 64))).to(device)
        self.graphs = {}

    def reset(self):
        self.ctl.zero_()
        self.log.zero_()
        for L in self.layers:
            if L["type"] == "linear_attention":
                L["ring"].zero_()
                L["S"].zero_()

    # ------------------------------------------------------------------ one pass of n rows
    def _layer(self, L, n, first):
        C, h, xn, mo = qa._C, self.h[:n], self.xn[:n], self.mo[:n]
        C.rmsnorm1p(h, None if first else mo, L["in_norm"], xn, self.eps)
        if L["type"] == "linear_attention":
            pr = self.proj[:n, :self.gdn_n]
            C.gemv_bf16(L["in_proj"], xn, pr)
            c0, c1, hv = self.conv_dim, self.conv_dim + self.hv * 128, self.hv
            out = self.mix[:n, :hv * 128]
            C.gdn_step_n(pr[:, :c0], pr[:, c0:c1], pr[:, c1:c1 + hv], pr[:, c1 + hv:], L["ring"],
                         L["conv_w"], L["A_log"], L["dt_bias"], L["norm_w"], L["S"], *L["st"],
                         self.ctl, out, self.hk, self.eps)
        else:
            pr = self.proj[:n, :self.attn_n]
            C.gemv_bf16(L["in_proj"], xn, pr)
            q0 = self.hq * 2 * HD
            k1 = q0 + self.hkv * HD
            qg, q = pr[:, :q0], self.q[:n]
            C.attn_prep(qg, pr[:, q0:k1], pr[:, k1:], L["q_norm"], L["k_norm"], self.inv_freq,
                        self.ctl, q, L["kc"], L["vc"], self.eps)
            out = self.mix[:n, :self.hq * HD]
            C.attn_decode(q, L["kc"], L["vc"], self.ctl, qg, self.part_o, self.part_ml, out)
        C.gemv_bf16(L["out"], out, mo)
        C.rmsnorm1p(h, mo, L["post_norm"], xn, self.eps)
        C.gemv_bf16(L["gate_up"], xn, self.gu[:n])
        C.swiglu(self.gu[:n], self.act[:n])
        C.gemv_bf16(L["down"], self.act[:n], mo)

    def _pass(self, n, k):
        C = qa._C
        C.embed(self.embed_t, self.in_tok, self.h[:n])
        for i, L in enumerate(self.layers):
            self._layer(L, n, i == 0)
        C.rmsnorm1p(self.h[:n], self.mo[:n], self.final_norm, self.hid[:n], self.eps)
        C.gemv_bf16(self.lm_head, self.hid[:n], self.logits[:n])
        C.argmax(self.logits[:n], self.am_v[:n * 256], self.am_i[:n * 256], self.am)
        C.accept(self.in_tok, self.am, n, self.ctl, self.next_tok, self.log)
        C.commit(self.ctl, self.in_tok, self.am, self.drafts, k)

    def _mutable(self):
        """Device state a pass changes: bookkeeping, and the recurrent layers' ring, state and
        staged rows (a pass replays staged rows into S, so a warm-up pass must be undone)."""
        out = [self.ctl, self.in_tok, self.log]
        for L in self.layers:
            if L["type"] == "linear_attention":
                out += [L["ring"], L["S"], *L["st"]]
        return out

    def graph(self, n, k):
        """The whole pass of n rows (k drafts staged for the next one) as one hipGraph."""
        if (n, k) not in self.graphs:
            saved = [t.clone() for t in self._mutable()]
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self._pass(n, k)  # warm-up outside capture (its state changes are undone below)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            for t, s in zip(self._mutable(), saved):
                t.copy_(s)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._pass(n, k)
            self.graphs[(n, k)] = g
        return self.graphs[(n, k)]

    # ------------------------------------------------------------------ generation loops
    def prefill(self, prompt: list[int]):
        """The prompt in one prefill pass (mode 0); its last row yields the first new token."""
        n = len(prompt)
        assert 1 <= n <= NMAX
        self.reset()
        self.in_tok[: n + 1] = torch.tensor(prompt + [-1], dtype=I32)
        self._pass(n, 0)
        self.ctl[2] = 1  # decode / verify from now on

    def generate_plain(self, prompt: list[int], n_new: int) -> list[int]:
        """Greedy decoding, one token per graph replay."""
        self.prefill(prompt)
        g = self.graph(1, 0)
        for _ in range(n_new - 1):
            g.replay()
        torch.cuda.synchronize()
        P = len(prompt)
        return self.log[P: P + n_new].tolist()

    def generate_spec(self, prompt: list[int], n_new: int, drafter, k: int = 3):
        """Verify passes of k + 1 rows; drafter(pos, last_token) gives k draft tokens for the next
        pass (a host function: the test controls how many drafts are right)."""
        self.prefill(prompt)
        P = len(prompt)
        g = self.graph(k + 1, k)
        passes = 0
        while True:
            torch.cuda.synchronize()
            pos = int(self.ctl[0])
            if pos + 1 >= P + n_new:
                break
            d = drafter(pos, int(self.in_tok[0]))
            self.in_tok[1: k + 1] = torch.tensor(d, dtype=I32)
            self.drafts[:k] = torch.tensor(d, dtype=I32)  # (commit copies these; overwritten above)
            g.replay()
            passes += 1
        torch.cuda.synchronize()
        return self.log[P: P + n_new].tolist(), passes, self.ctl.tolist()
