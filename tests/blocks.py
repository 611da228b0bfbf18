"""Bottleneck blocks with SpikingJelly's attribute names, for the
substitution and parity tests of CTFSEWBottleneck / CTFSpikingBottleneck
(catfuse/substitute.py matches them by class name "Bottleneck" and by the
presence of `cnf`, as SpikingJelly's sew_resnet / spiking_resnet
Bottlenecks differ)."""
import torch.nn as nn

from catfuse_amd import snn


class SEWBottleneck(nn.Module):
    """SEW-ResNet Bottleneck: 1x1 -> 3x3 (stride) -> 1x1, each Conv-BN-LIF,
    then sew(identity, out); identity = downsample_sn(downsample(x)) or x."""
    expansion = 4

    def __init__(self, inplanes, planes, stride=1, cnf="ADD", downsample=False):
        super().__init__()
        width = planes
        self.conv1 = snn.Conv2d(inplanes, width, 1, 1, 0, bias=False)
        self.bn1 = snn.BatchNorm2d(width)
        self.sn1 = snn.LIFNode()
        self.conv2 = snn.Conv2d(width, width, 3, stride, 1, bias=False)
        self.bn2 = snn.BatchNorm2d(width)
        self.sn2 = snn.LIFNode()
        self.conv3 = snn.Conv2d(width, planes * self.expansion, 1, 1, 0, bias=False)
        self.bn3 = snn.BatchNorm2d(planes * self.expansion)
        self.sn3 = snn.LIFNode()
        self.downsample = None
        if downsample:
            self.downsample = nn.Sequential(
                snn.Conv2d(inplanes, planes * self.expansion, 1, stride, 0, bias=False),
                snn.BatchNorm2d(planes * self.expansion))
            self.downsample_sn = snn.LIFNode()
        self.stride = stride
        self.cnf = cnf

    def forward(self, x):
        out = self.sn1(self.bn1(self.conv1(x)))
        out = self.sn2(self.bn2(self.conv2(out)))
        out = self.sn3(self.bn3(self.conv3(out)))
        identity = x if self.downsample is None else self.downsample_sn(self.downsample(x))
        return snn.sew_function(identity, out, self.cnf)


class SpikingBottleneck(nn.Module):
    """Spiking-ResNet Bottleneck (no cnf): LIF(BN(conv3(.)) + identity),
    identity = BN(conv_ds(x)) or x."""
    expansion = 4

    def __init__(self, inplanes, planes, stride=1, downsample=False):
        super().__init__()
        width = planes
        self.conv1 = snn.Conv2d(inplanes, width, 1, 1, 0, bias=False)
        self.bn1 = snn.BatchNorm2d(width)
        self.sn1 = snn.LIFNode()
        self.conv2 = snn.Conv2d(width, width, 3, stride, 1, bias=False)
        self.bn2 = snn.BatchNorm2d(width)
        self.sn2 = snn.LIFNode()
        self.conv3 = snn.Conv2d(width, planes * self.expansion, 1, 1, 0, bias=False)
        self.bn3 = snn.BatchNorm2d(planes * self.expansion)
        self.sn3 = snn.LIFNode()
        self.downsample = None
        if downsample:
            self.downsample = nn.Sequential(
                snn.Conv2d(inplanes, planes * self.expansion, 1, stride, 0, bias=False),
                snn.BatchNorm2d(planes * self.expansion))

    def forward(self, x):
        out = self.sn1(self.bn1(self.conv1(x)))
        out = self.sn2(self.bn2(self.conv2(out)))
        out = self.bn3(self.conv3(out))
        identity = x if self.downsample is None else self.downsample(x)
        return self.sn3(out + identity)


SEWBottleneck.__name__ = "Bottleneck"
SpikingBottleneck.__name__ = "Bottleneck"
