"""Network definitions the layer tests convert (plain torch; torchvision is not installed).

``resnet18`` is ResNet-18 (BasicBlock [2, 2, 2, 2], 1000 classes) with
Kaiming-normal convolution weights, for BASELINE config 4.  ``LeNet5`` is the
architecture of memfast/models/lenet.py:6-28 (two 5x5 convolutions with tanh
and average pooling, three linear layers), whose shipped static-INT4
checkpoint the checkpoint tests load.
"""

from torch import nn


class _Block(nn.Module):
    def __init__(self, cin, cout, stride):
        super().__init__()
        self.conv1 = nn.Conv2d(cin, cout, 3, stride, 1, bias=False)
        self.bn1 = nn.BatchNorm2d(cout)
        self.conv2 = nn.Conv2d(cout, cout, 3, 1, 1, bias=False)
        self.bn2 = nn.BatchNorm2d(cout)
        self.down = None
        if stride != 1 or cin != cout:
            self.down = nn.Sequential(nn.Conv2d(cin, cout, 1, stride, bias=False),
                                      nn.BatchNorm2d(cout))

    def forward(self, x):
        out = self.bn1(self.conv1(x)).relu()
        out = self.bn2(self.conv2(out))
        return (out + (x if self.down is None else self.down(x))).relu()


def resnet18(classes=1000):
    layers = [nn.Conv2d(3, 64, 7, 2, 3, bias=False), nn.BatchNorm2d(64), nn.ReLU(),
              nn.MaxPool2d(3, 2, 1)]
    cin = 64
    for cout, stride in ((64, 1), (128, 2), (256, 2), (512, 2)):
        layers += [_Block(cin, cout, stride), _Block(cout, cout, 1)]
        cin = cout
    layers += [nn.AdaptiveAvgPool2d(1), nn.Flatten(), nn.Linear(512, classes)]
    model = nn.Sequential(*layers)
    for module in model.modules():
        if isinstance(module, nn.Conv2d):
            nn.init.kaiming_normal_(module.weight, mode="fan_out", nonlinearity="relu")
    return model.eval()


class LeNet5(nn.Module):
    """Module names match the shipped checkpoints' state-dict prefixes
    (``features.0``, ``features.3``, ``classifier.0/2/4``)."""

    def __init__(self, classes=10):
        super().__init__()
        self.features = nn.Sequential(
            nn.Conv2d(1, 6, 5, padding=2), nn.Tanh(), nn.AvgPool2d(2),
            nn.Conv2d(6, 16, 5), nn.Tanh(), nn.AvgPool2d(2),
        )
        self.classifier = nn.Sequential(
            nn.Linear(16 * 5 * 5, 120), nn.Tanh(), nn.Linear(120, 84), nn.Tanh(),
            nn.Linear(84, classes),
        )

    def forward(self, x):
        return self.classifier(self.features(x).flatten(1))
