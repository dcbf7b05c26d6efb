"""Build tests/golden/unet_segment_20steps.npz from the reference's own data.

The reference holds one record of its engine's outputs on the training path:
compare_result.log (UTF-16), 20 lock-step UNet-base16 training steps at
128x128, batch 2, produced by compare_unet_20batch.py.  This script restates
that run's inputs as a small fixture:

* the 40 images/masks the 20 batches use: segment/png_images/IMAGES and
  segment/png_masks/MASKS sorted by name, resized to 128x128 with Pillow's
  default filter, images as uint8 RGB, masks binarised (> 0.01 after /255),
  batches = np.random.seed(0) permutation of the 1000 samples taken two at a
  time (compare_unet_20batch.py:24-36, :287-292);
* the logged DirectCompute loss and gradient norm of each step
  (compare_result.log:14-33, columns "DC Loss" and "DC Norm").

Initial weights are not stored: they are np.random.RandomState(42) draws that
the tests regenerate (compare_unet_20batch.py:38-63).

Run from the repository root:  python tests/golden/make_unet_segment_fixture.py
"""
import glob
import os

import numpy as np
from PIL import Image

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "unet_segment_20steps.npz")
IMG = 128
STEPS, BATCH = 20, 2


def parse_log():
    text = open(os.path.join(REF, "compare_result.log"), "rb").read().decode("utf-16")
    loss, norm = [], []
    for line in text.splitlines():
        parts = line.replace("|", " ").split()
        if len(parts) >= 8 and parts[0].isdigit() and 1 <= int(parts[0]) <= STEPS:
            loss.append(float(parts[2]))      # DC Loss
            norm.append(float(parts[5]))      # DC Norm
    assert len(loss) == STEPS, len(loss)
    return np.array(loss), np.array(norm)


def main():
    imgs = sorted(glob.glob(os.path.join(REF, "segment", "png_images", "IMAGES", "*.png")) +
                  glob.glob(os.path.join(REF, "segment", "png_images", "IMAGES", "*.jpg")))
    masks = sorted(glob.glob(os.path.join(REF, "segment", "png_masks", "MASKS", "*.png")) +
                   glob.glob(os.path.join(REF, "segment", "png_masks", "MASKS", "*.jpg")))
    assert len(imgs) == len(masks) == 1000
    np.random.seed(0)
    perm = np.random.permutation(len(imgs))
    order = perm[: STEPS * BATCH]
    X = np.empty((len(order), IMG, IMG, 3), np.uint8)
    Y = np.empty((len(order), IMG, IMG), np.bool_)
    for j, i in enumerate(order):
        X[j] = np.array(Image.open(imgs[i]).convert("RGB").resize((IMG, IMG)), dtype=np.uint8)
        m = np.array(Image.open(masks[i]).convert("L").resize((IMG, IMG)), dtype=np.float32) / 255.0
        Y[j] = m > 0.01
    loss, norm = parse_log()
    np.savez_compressed(OUT, images_u8=X, masks=np.packbits(Y, axis=-1), sample_index=order,
                        dc_loss=loss, dc_norm=norm)
    print(f"wrote {OUT} ({os.path.getsize(OUT) / 1e6:.2f} MB)")


if __name__ == "__main__":
    main()
