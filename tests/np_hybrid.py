"""Float64 numpy restatement of the qwen35 hybrid decode step, written from the
reference's source independently of the C oracle:

* Gated-DeltaNet layer, qwen35.rs:1239-1492 (conv window qwen35.rs:264-315,
  depthwise_conv :1820-1829, softplus :1809-1815).  Per v-head h with k-group
  h % n_groups: dot_j = sum_i S[i][j] k_i on the UNDECAYED state, then
  S[i][j] = S[i][j]*exp(g) + k_i*beta*(v_j - dot_j), o_j = sum_i S[i][j] q_i / sqrt(hd).
* Gated full-attention layer, qwen35.rs:1495-1640: attn_q emits [q_h | gate_h]
  per head, head RMSNorms, partial NeoX RoPE on the first rope_dim dims
  (ops.rs:78-164), GQA with kv head qh / (n_heads / n_kv), o / (1 + exp(-gate)).
* Layer composition and FFN, qwen35.rs:1028-1236.

Every matmul input is Q8_0-quantized first (the `mm` path), so the projections
use the dequantized Q8_0 activation; alpha/beta read the f32 normed hidden.

`mutate` names one deliberate mistake, used to show that a comparison against
this restatement can tell the mistake apart:
  "decay_before_dot"  the dot reads the decayed state
  "state_transposed"  the dot reads S[j][i] while the update writes S[i][j]
  "gate_from_q"       the sigmoid gate read from the q half of each head
  "no_conv_history"   the conv window forgets earlier tokens
  "khead_div"         v-head h pairs with k-group h // rep instead of h % n_groups
  "rope_full"         RoPE rotates the whole head instead of the first rope_dim dims
  "no_qk_norm"        the q/k head RMSNorms are skipped
  "no_ssm_perm"       (folded models) ssm_out's input is rotated without the
                      grouped head permutation
  "unrotate_as_rotate" (folded models) the latent embedding row gets R instead of R^-1

Folded models (cfg.had_block > 0, qwen35.rs:51-118, :881-970): every matmul
input x is quantized as R x = WHT_b(signs * x) (normalized Sylvester WHT per
block, scipy.linalg.hadamard / sqrt(b)); ssm_out's input is first permuted to
grouped head order (qwen35.rs:1452-1478); a latent embedding row gets
R^-1 = H D (WHT, then signs); a tied head reads token_embd.
"""
import numpy as np

from fixtures import np_dequant


class NpHybrid:
    def __init__(self, oracle_model, cfg, mutate=None, signs=None):
        self.m, self.c, self.mut = oracle_model, cfg, mutate
        self.signs = signs or {}
        c = cfg
        self.hd = c.ssm_head_dim
        self.nk, self.nv = c.ssm_n_k_heads, c.ssm_n_v_heads
        self.kdim, self.vdim = self.nk * self.hd, self.nv * self.hd
        self.conv_dim = 2 * self.kdim + self.vdim
        self.K = c.ssm_conv_kernel
        self.rope_dim = c.rope_dim or c.head_dim
        self._cache = {}
        self.reset()

    def reset(self):
        c = self.c
        self.S = {i: np.zeros((self.nv, self.hd, self.hd)) for i in range(c.n_layers)}
        self.win = {i: np.zeros((self.K - 1, self.conv_dim)) for i in range(c.n_layers)}
        self.kc = {i: [] for i in range(c.n_layers)}
        self.vc = {i: [] for i in range(c.n_layers)}

    # ---- tensors
    def W(self, name, rows, cols, t=None):
        key = (name, t)
        if key not in self._cache:
            t = self.c.wtype if t is None else t
            self._cache[key] = np_dequant(t, self.m.tensor(name), rows * cols).reshape(rows, cols).astype(np.float64)
        return self._cache[key]

    def F(self, name):
        return self.m.tensor(name).view(np.float32).astype(np.float64)

    def rms(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.c.eps) * w

    def q8(self, x):
        from oracle import oracle as orc
        return np_dequant(8, orc.quantize_q8_0(x.astype(np.float32)), x.size).astype(np.float64)

    def wht(self, x):
        import scipy.linalg
        b = self.c.had_block
        H = scipy.linalg.hadamard(b).astype(np.float64) / np.sqrt(b)
        return (x.reshape(-1, b) @ H.T).reshape(-1)

    def mmq(self, x):
        """The Q8_0 activation a matmul sees: x, or R x on a folded model."""
        if self.c.had_block:
            sg = self.signs.get(x.size)
            x = self.wht(x * sg if sg is not None else x)
        return self.q8(x)

    @staticmethod
    def silu(z):
        return z / (1 + np.exp(-z))

    def rope(self, x, pos):
        c, rd = self.c, (self.c.head_dim if self.mut == "rope_full" else self.rope_dim)
        half = rd // 2
        inv = 1.0 / c.rope_theta ** (2.0 * np.arange(half) / rd)
        f = pos * inv
        s, co = np.sin(f), np.cos(f)
        y = x.copy()
        x0, x1 = x[:half], x[half:rd]
        y[:half] = x0 * co - x1 * s
        y[half:rd] = x0 * s + x1 * co
        return y

    # ---- layers
    def gdn(self, i, nrm, x):
        c, hd, nk, nv = self.c, self.hd, self.nk, self.nv
        kdim, vdim, K = self.kdim, self.vdim, self.K
        p = f"blk.{i}."
        qkv = self.W(p + "attn_qkv.weight", self.conv_dim, c.d_model) @ x
        z = self.W(p + "attn_gate.weight", vdim, c.d_model) @ x
        a = self.F(p + "ssm_alpha.weight").reshape(nv, c.d_model) @ nrm
        b = self.F(p + "ssm_beta.weight").reshape(nv, c.d_model) @ nrm
        if self.mut == "no_conv_history":
            self.win[i][:] = 0
        window = np.vstack([self.win[i], qkv[None, :]])          # [K][ch], tap K-1 = current
        self.win[i] = window[1:]
        cw = self.F(p + "ssm_conv1d.weight").reshape(self.conv_dim, K)
        co = self.silu((cw * window.T).sum(1))
        qh = co[:kdim].reshape(nk, hd)
        kh = co[kdim:2 * kdim].reshape(nk, hd)
        qh = qh / np.sqrt((qh * qh).sum(1, keepdims=True) + c.eps)
        kh = kh / np.sqrt((kh * kh).sum(1, keepdims=True) + c.eps)
        v = co[2 * kdim:].reshape(nv, hd)
        sp = a + self.F(p + "ssm_dt.bias")
        sp = np.where(sp > 20, sp, np.log1p(np.exp(sp)))
        g = sp * self.F(p + "ssm_a")
        beta = 1 / (1 + np.exp(-b))
        rep = nv // nk
        o = np.zeros((nv, hd))
        for h in range(nv):
            kg = h // rep if self.mut == "khead_div" else h % nk
            S = self.S[i][h]
            decay = np.exp(g[h])
            if self.mut == "decay_before_dot":
                S = S * decay
                dot = S.T @ kh[kg]
                S = S + np.outer(kh[kg], beta[h] * (v[h] - dot))
            else:
                dot = S.T @ kh[kg]                                # dot_j = sum_i S[i][j] k_i
                if self.mut == "state_transposed":
                    dot = S @ kh[kg]
                S = S * decay + np.outer(kh[kg], beta[h] * (v[h] - dot))
            o[h] = S.T @ qh[kg] / np.sqrt(hd)
            self.S[i][h] = S
        on = np.stack([self.rms(o[h], self.F(p + "ssm_norm.weight")) for h in range(nv)]).reshape(-1)
        on = on * self.silu(z)
        if self.c.had_block and nv // nk > 1 and self.mut != "no_ssm_perm":
            rep = nv // nk
            perm = np.zeros_like(on)
            for h in range(nv):
                dst = ((h % nk) * rep + h // nk) * hd
                perm[dst:dst + hd] = on[h * hd:(h + 1) * hd]
            on = perm
        return self.W(p + "ssm_out.weight", c.d_model, vdim) @ self.mmq(on)

    def attn(self, i, x, pos):
        c, hd = self.c, self.c.head_dim
        nh, nkv = c.n_heads, c.n_kv_heads
        p = f"blk.{i}."
        qg = self.W(p + "attn_q.weight", 2 * nh * hd, c.d_model) @ x
        k = self.W(p + "attn_k.weight", nkv * hd, c.d_model) @ x
        v = self.W(p + "attn_v.weight", nkv * hd, c.d_model) @ x
        qg = qg.reshape(nh, 2, hd)
        q, gate = qg[:, 0], qg[:, 1]
        if self.mut == "gate_from_q":
            gate = qg[:, 0]
        qn, kn = self.F(p + "attn_q_norm.weight"), self.F(p + "attn_k_norm.weight")
        if self.mut == "no_qk_norm":
            self.rms = lambda x, w: x
        q = np.stack([self.rope(self.rms(q[h], qn), pos) for h in range(nh)])
        k = np.stack([self.rope(self.rms(k.reshape(nkv, hd)[h], kn), pos) for h in range(nkv)])
        if self.mut == "no_qk_norm":
            del self.rms
        self.kc[i].append(k)
        self.vc[i].append(v.reshape(nkv, hd))
        Kc, Vc = np.stack(self.kc[i], 1), np.stack(self.vc[i], 1)      # [kv][t][hd]
        out = np.zeros((nh, hd))
        for h in range(nh):
            kvh = h // (nh // nkv)
            s = Kc[kvh] @ q[h] / np.sqrt(hd)
            e = np.exp(s - s.max())
            out[h] = (e / e.sum()) @ Vc[kvh]
        out = out / (1 + np.exp(-gate))
        return self.W(p + "attn_output.weight", c.d_model, nh * hd) @ self.mmq(out.reshape(-1))

    def forward(self, tok, pos):
        c, d = self.c, self.c.d_model
        h = self.W("token_embd.weight", c.vocab, d, 8)[tok].copy()
        if c.had_block and (c.had_flags & 1):
            sg = self.signs.get(d)
            if self.mut == "unrotate_as_rotate":
                h = self.wht(h * sg if sg is not None else h)
            else:
                h = self.wht(h)
                h = h * sg if sg is not None else h
        for i in range(c.n_layers):
            p = f"blk.{i}."
            nrm = self.rms(h, self.F(p + "attn_norm.weight"))
            x = self.mmq(nrm)
            if (i + 1) % c.full_attn_interval != 0:
                h = h + self.gdn(i, nrm, x)
            else:
                h = h + self.attn(i, x, pos)
            x = self.mmq(self.rms(h, self.F(p + "post_attention_norm.weight")))
            g = self.W(p + "ffn_gate.weight", c.d_ffn, d) @ x
            u = self.W(p + "ffn_up.weight", c.d_ffn, d) @ x
            h = h + self.W(p + "ffn_down.weight", d, c.d_ffn) @ self.mmq(self.silu(g) * u)
        x = self.mmq(self.rms(h, self.F("output_norm.weight")))
        head = "token_embd.weight" if (c.had_block and (c.had_flags & 2)) else "output.weight"
        return self.W(head, c.vocab, d, 8) @ x
