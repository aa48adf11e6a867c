"""End-to-end training harness: the reference's ``train.py`` network on dcnv2_amd.

The network is the reference's ResNet with 1x1 deformable convolutions
(``train.py:51-108``: ``Resblock``, ``Add_module1`` and the (3, 4, 23, 3)-block
``net`` with a 10-way head), trained with the reference's step (Adam, lr 1e-4,
betas (0.9, 0.999), eps 1e-8, cross-entropy; ``train.py:137-163``).  CIFAR-10 is
not downloadable here, so the data are synthetic: seeded random 3x224x224
images (the reference resizes CIFAR-10 to 224, ``train.py:14-29``) and random
labels.  ``MyDCN`` is ``dcnv2_amd.DCN`` (the reference imports
``dcn_v2_mm.DCN as MyDCN``, ``train.py:12``).

Usage: ``python train.py [--steps K] [--batch B] [--size S] [--depths 3,4,23,3]``
prints one JSON line with the step time; ``build_net`` is shared with the tests.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch
import torch.nn as nn
import torch.optim as optim

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

from dcnv2_amd.dcn_v2_mm import DCN as MyDCN  # noqa: E402


class Resblock(nn.Sequential):
    """Reference ``train.py:51-77``: 1x1 DCN -> BN -> 3x3 conv -> BN -> 1x1 DCN ->
    BN -> ReLU, plus a shortcut (1x1 DCN and max-pool when strided)."""

    def __init__(self, in_channels, num_kernel, out_channels, stride, dcn=MyDCN):
        super().__init__()
        self.m1 = nn.Sequential(
            dcn(in_channels, num_kernel, kernel_size=1, padding=0),
            nn.BatchNorm2d(num_kernel),
            nn.Conv2d(num_kernel, num_kernel, kernel_size=3, stride=stride, padding=1),
            nn.BatchNorm2d(num_kernel),
            dcn(num_kernel, out_channels, kernel_size=1, padding=0),
            nn.BatchNorm2d(out_channels),
            nn.ReLU(),
        )
        if stride == 2:
            self.m2 = nn.Sequential(dcn(in_channels, out_channels, kernel_size=1, padding=0),
                                    nn.MaxPool2d(kernel_size=2, stride=stride))
        elif in_channels == out_channels:
            self.m2 = nn.Sequential()
        else:
            self.m2 = nn.Sequential(dcn(in_channels, out_channels, kernel_size=1, padding=0))

    def forward(self, x):
        return self.m1(x) + self.m2(x)


class Add_module1(nn.Sequential):
    """Reference ``train.py:79-91``: n Resblocks, the first with stride 2."""

    def __init__(self, n, in_channels, num_kernel, out_channels, dcn=MyDCN):
        super().__init__()
        self.m3 = nn.Sequential()
        for i in range(n):
            cin = in_channels if i == 0 else out_channels
            self.m3.add_module(str(i), Resblock(cin, num_kernel, out_channels,
                                                stride=2 if i == 0 else 1, dcn=dcn))

    def forward(self, x):
        return self.m3(x)


def build_net(depths=(3, 4, 23, 3), num_classes=10, dcn=MyDCN) -> nn.Sequential:
    """The reference's ``net`` (``train.py:94-108``); ``depths`` = (leading
    Resblocks, then the blocks of the three Add_module1 stages)."""
    d0, d1, d2, d3 = depths
    layers = [nn.Conv2d(3, 64, kernel_size=7, stride=2, padding=3), nn.BatchNorm2d(64), nn.ReLU(),
              nn.MaxPool2d(kernel_size=3, stride=2, padding=1),
              Resblock(64, 64, 256, 1, dcn=dcn)]
    layers += [Resblock(256, 64, 256, 1, dcn=dcn) for _ in range(d0 - 1)]
    layers += [Add_module1(d1, 256, 128, 512, dcn=dcn), Add_module1(d2, 512, 256, 1024, dcn=dcn),
               Add_module1(d3, 1024, 512, 2048, dcn=dcn),
               nn.AdaptiveAvgPool2d(output_size=(1, 1)), nn.Flatten(),
               nn.Linear(in_features=2048, out_features=num_classes)]
    return nn.Sequential(*layers)


def synthetic_batch(batch, size, num_classes=10, seed=0, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(batch, 3, size, size, generator=g)
    y = torch.randint(0, num_classes, (batch,), generator=g)
    return x.to(device), y.to(device)


def train_step(net, optimizer, criterion, x, y):
    """One step of the reference's loop body (``train.py:145-151``)."""
    optimizer.zero_grad()
    loss = criterion(net(x), y)
    loss.backward()
    optimizer.step()
    return loss.detach()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--batch", type=int, default=128)
    ap.add_argument("--size", type=int, default=224)
    ap.add_argument("--depths", default="3,4,23,3")
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    depths = tuple(int(v) for v in args.depths.split(","))
    torch.manual_seed(0)
    net = build_net(depths).to(dev)
    optimizer = optim.Adam(net.parameters(), betas=(0.9, 0.999), eps=1e-08, lr=1e-4,
                           amsgrad=False)
    criterion = nn.CrossEntropyLoss()
    x, y = synthetic_batch(args.batch, args.size, device=dev)
    net.train()
    for _ in range(args.warmup):
        train_step(net, optimizer, criterion, x, y)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    losses = [float(train_step(net, optimizer, criterion, x, y)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    n_dcn = sum(isinstance(m, MyDCN) for m in net.modules())
    print(json.dumps({"workload": f"reference train.py net, depths {depths}, {n_dcn} DCN layers, "
                                  f"batch {args.batch}, {args.size}x{args.size}, fp32, synthetic",
                      "ms_per_step": round(ms, 2), "images_per_s": round(args.batch * 1e3 / ms, 1),
                      "losses": [round(v, 4) for v in losses]}), flush=True)


if __name__ == "__main__":
    main()
