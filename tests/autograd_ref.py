"""An independent float64 statement of the relaxation through torch autograd.

The reference's state update (Layer.cs:273-309) is gradient descent on the
free energy
    F = sum_{l=0}^{L-2} 0.5 * P_l * |mu_l - f(W_{l+1} mu_{l+1} + b_{l+1})|^2
        + lambda * sum_{l>=1} |mu_l|
with step eta: dF/dmu_l = e_l - W_l^T (f'(pre_l) . e_{l-1}) + lambda*sign(mu_l).
Here torch derives that gradient itself from F, so a dropped term, a wrong
sign, a transposed weight or a wrong f' in the oracle fails against it.
Energies are F without the lambda term, at the pre-update state of each step
(Network.cs:876-907 reads energy after UpdateState from the errors computed
before it).
"""
import numpy as np
import torch
import torch.nn.functional as Fn


def _act(name):
    return {
        "linear": lambda x: x,
        "tanh": torch.tanh,
        "relu": torch.relu,
        "sigmoid": torch.sigmoid,
        "gelu": lambda x: Fn.gelu(x, approximate="tanh"),
    }[name]


def autograd_relax(sizes, act, eta, W, b, prec, x0, steps, act_reg=0.0, ffg=False, top_clamp=None,
                   want_delta=False, init_hidden=None):
    """Settles from zero hidden states (or from init_hidden, a list of [B, s_l]
    arrays for l = 1..L-2); with top_clamp [B, s_top] the top layer is held
    there (not a free variable).  With want_delta it also returns, for every
    layer l >= 1, delta_l = -dF/dpre_l at the last step's pre-update state
    (autograd through the pre-activation itself)."""
    f = _act(act)
    L = len(sizes)
    dt = torch.float64
    Wt = [torch.tensor(np.asarray(w, dtype=np.float64), dtype=dt) for w in W]
    bt = [torch.tensor(np.asarray(v, dtype=np.float64), dtype=dt) for v in b]
    P = [float(p) for p in prec]
    x = torch.tensor(np.asarray(x0, dtype=np.float64), dtype=dt)
    B = x.shape[0]
    mu = [x] + [torch.zeros(B, s, dtype=dt) for s in sizes[1:]]
    if init_hidden is not None:
        for l, h in enumerate(init_hidden, start=1):
            mu[l] = torch.tensor(np.asarray(h, dtype=np.float64), dtype=dt).reshape(B, sizes[l])
    nfree = L - 1
    if top_clamp is not None:
        mu[-1] = torch.tensor(np.asarray(top_clamp, dtype=np.float64), dtype=dt).reshape(B, sizes[-1])
        nfree = L - 2
    if ffg:
        for l in range(L - 1, 0, -1):
            pred = f(mu[l] @ Wt[l - 1].T + bt[l - 1])
            if l > 1:
                mu[l - 1] = pred.detach().clone()
    energies = np.zeros((steps, B))
    deltas = None
    for t in range(steps):
        free = [m.clone().requires_grad_(True) for m in mu[1:1 + nfree]]
        full = [mu[0]] + free + mu[1 + nfree:]
        Fb = torch.zeros(B, dtype=dt)
        pres = []
        for l in range(L - 1):
            pre = full[l + 1] @ Wt[l].T + bt[l]
            if want_delta and t == steps - 1:
                if pre.requires_grad:
                    pre.retain_grad()
                else:   # the clamped top's pre-activation: a leaf of its own
                    pre = pre.detach().requires_grad_(True)
            pres.append(pre)
            r = full[l] - f(pre)
            Fb = Fb + 0.5 * P[l] * (r * r).sum(dim=1)
        energies[t] = Fb.detach().numpy()
        F = Fb.sum()
        if act_reg > 0:
            F = F + act_reg * sum(m.abs().sum() for m in free)
        if want_delta and t == steps - 1:
            F.backward()
            grads = [m.grad for m in free]
            deltas = [None] + [(-p.grad).numpy() for p in pres]
        else:
            grads = torch.autograd.grad(F, free) if free else []
        mu = [mu[0]] + [(m - eta * g).detach() for m, g in zip(free, grads)] + mu[1 + nfree:]
    if want_delta:
        return mu[-1].numpy(), [m.numpy() for m in mu], energies, deltas
    return mu[-1].numpy(), [m.numpy() for m in mu], energies


def autograd_learn(sizes, act, eta, W, b, prec, x0, labels, steps, eta_w, weight_decay=0.0, init_hidden=None,
                   want_hidden=False):
    """Learning step from the autograd settling: W_l += eta_w delta_l^T mu_l
    (settled mu_l), b_l += eta_w sum delta_l, then W_l -= eta_w lambda W_l.
    The settling starts from init_hidden (zeros if None); with want_hidden the
    settled hidden states come back too."""
    _, mus, energies, deltas = autograd_relax(sizes, act, eta, W, b, prec, x0, steps, top_clamp=labels,
                                              want_delta=True, init_hidden=init_hidden)
    new_w, new_b = [], []
    for l in range(1, len(sizes)):
        w = np.asarray(W[l - 1], dtype=np.float64) + eta_w * deltas[l].T @ mus[l]
        bb = np.asarray(b[l - 1], dtype=np.float64) + eta_w * deltas[l].sum(axis=0)
        if weight_decay > 0:
            w = w - eta_w * weight_decay * w
        new_w.append(w)
        new_b.append(bb)
    if want_hidden:
        return new_w, new_b, energies[-1], mus[1:-1]
    return new_w, new_b, energies[-1]


ROUND_POINTS = ("state", "wt", "delta", "w")


def _round16(x, mode):
    """Round-to-nearest-even to bf16 or fp16 of the fp32 value of x (torch's
    own conversions), carried on in float64."""
    if mode == "bf16":
        return x.float().to(torch.bfloat16).double()
    return x.float().to(torch.float16).double()


def mixed_relax_f64(sizes, act, eta, W, b, prec, x0, steps, mode, drop=()):
    """The batched relaxation with 16-bit GEMM operands, stated directly in
    float64: every operation in float64 except that both operands of both
    GEMMs are rounded to `mode` where BatchedPcForward's mixed path rounds them
    (Gemm.cs:44-60 rounds A and B of every MatMulMixed call):
        pre_l = round(M_l) round(W_l)^T + b_l            (TopDown, :74-80)
        G_l   = round(f'(pre_l) * e_{l-1}) round(W_l)     (Mul(delta, W_l), :117)
    The weights never change during a settling, so rounding them once equals
    rounding them per call.  `drop` names rounding points to leave out
    ("state", "wt", "delta", "w"): each one left out moves the result by far
    more than the fp32-versus-float64 difference, which is how a test shows
    that this statement pins every point.  Returns (top, energies [T, B])."""
    f = _act(act)
    fprime = _act_deriv(act)
    dt = torch.float64
    L = len(sizes)
    R = lambda x, point: x if point in drop else _round16(x, mode)
    Wt = [torch.tensor(np.asarray(w, dtype=np.float64), dtype=dt) for w in W]
    W_g2 = [R(w, "w") for w in Wt]               # GEMM 2's B operand, W_l
    W_g1 = [R(w.T.contiguous(), "wt") for w in Wt]  # GEMM 1's B operand, W_l^T
    bt = [torch.tensor(np.asarray(v, dtype=np.float64), dtype=dt) for v in b]
    P = [float(p) for p in prec]
    x = torch.tensor(np.asarray(x0, dtype=np.float64), dtype=dt)
    B = x.shape[0]
    mu = [x] + [torch.zeros(B, s, dtype=dt) for s in sizes[1:]]
    energies = np.zeros((steps, B))
    for t in range(steps):
        pre = [None] + [R(mu[l], "state") @ W_g1[l - 1] + bt[l - 1] for l in range(1, L)]
        e = [P[l] * (mu[l] - f(pre[l + 1])) for l in range(L - 1)] + [torch.zeros(B, sizes[-1], dtype=dt)]
        energies[t] = sum(0.5 * (e[l] * e[l]).sum(dim=1) / P[l] for l in range(L - 1)).numpy()
        new = [mu[0]]
        for l in range(1, L):
            delta = fprime(pre[l]) * e[l - 1]
            g = R(delta, "delta") @ W_g2[l - 1]
            new.append(mu[l] - eta * (e[l] - g))
        mu = new
    return mu[-1].numpy(), energies


def _act_deriv(name):
    """f'(pre) in closed form, as Activation.cs:86-132 and Autograd.cs:313-318
    state them (tanh from the output, GELU-tanh from the pre-activation)."""
    def gelu_d(x):
        c, a = 0.7978845608028654, 0.044715
        t = torch.tanh(c * (x + a * x ** 3))
        return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * c * (1 + 3 * a * x * x)
    return {
        "linear": lambda x: torch.ones_like(x),
        "tanh": lambda x: 1 - torch.tanh(x) ** 2,
        "relu": lambda x: (x > 0).to(x.dtype),
        "sigmoid": lambda x: torch.sigmoid(x) * (1 - torch.sigmoid(x)),
        "gelu": gelu_d,
    }[name]
