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


def autograd_relax(sizes, act, eta, W, b, prec, x0, steps, act_reg=0.0, ffg=False):
    f = _act(act)
    L = len(sizes)
    dt = torch.float64
    Wt = [torch.tensor(np.asarray(w, dtype=np.float64), dtype=dt) for w in W]
    bt = [torch.tensor(np.asarray(v, dtype=np.float64), dtype=dt) for v in b]
    P = [float(p) for p in prec]
    x = torch.tensor(np.asarray(x0, dtype=np.float64), dtype=dt)
    B = x.shape[0]
    mu = [x] + [torch.zeros(B, s, dtype=dt) for s in sizes[1:]]
    if ffg:
        for l in range(L - 1, 0, -1):
            pred = f(mu[l] @ Wt[l - 1].T + bt[l - 1])
            if l > 1:
                mu[l - 1] = pred.detach().clone()
    energies = np.zeros((steps, B))
    for t in range(steps):
        free = [m.clone().requires_grad_(True) for m in mu[1:]]
        full = [mu[0]] + free
        Fb = torch.zeros(B, dtype=dt)
        for l in range(L - 1):
            r = full[l] - f(full[l + 1] @ Wt[l].T + bt[l])
            Fb = Fb + 0.5 * P[l] * (r * r).sum(dim=1)
        energies[t] = Fb.detach().numpy()
        F = Fb.sum()
        if act_reg > 0:
            F = F + act_reg * sum(m.abs().sum() for m in free)
        grads = torch.autograd.grad(F, free)
        mu = [mu[0]] + [(m - eta * g).detach() for m, g in zip(free, grads)]
    return mu[-1].numpy(), [m.numpy() for m in mu], energies
