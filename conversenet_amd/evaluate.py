"""Image-quality evaluation: PSNR / SSIM, image IO without OpenCV, the test-time degradations, and a
command line that runs the three test scripts' loops on a folder of images.

Follows the reference's evaluation path:
  * utils/utils_image.py: imread_uint (:189-201), imsave (:207-211), uint2single / single2uint
    (:253-259), single2tensor4 (:311-312), tensor2uint (:293-297), modcrop (:498-511),
    rgb2ycbcr (:533-558), calculate_psnr (:626-641), calculate_ssim / ssim (:647-696), imresize_np
    (MATLAB-style bicubic, antialiased when shrinking);
  * main_test_converse_dncnn.py:110-171 (gray denoising, AWGN with np.random.seed(0)),
    main_test_converse_srresnet.py:115-171 (modcrop, bicubic x1/sf, PSNR/SSIM with a border of sf,
    Y-channel scores), main_test_converse_usrnet.py:130-192 (modcrop to lcm(sf, 8), wrap blur with a
    kernel from blur_kernels/, s-fold decimation at offset 0, AWGN, PSNR with a border of sf^2).

Images are read and written with Pillow.  Gray conversion of colour files uses the ITU-R 601 weights
in OpenCV's 14-bit fixed point ((4899 R + 9617 G + 1868 B + 8192) >> 14); OpenCV's own imread may
decode some formats to gray inside the codec, which can differ by one level on a few pixels.
"""
import argparse
import glob
import math
import os

import numpy as np
import torch

IMG_EXTENSIONS = (".jpg", ".jpeg", ".png", ".ppm", ".bmp", ".tif", ".tiff")


# ---------------------------------------------------------------------------------------------
# IO and conversions
# ---------------------------------------------------------------------------------------------
def get_image_paths(root):
    """Sorted image files under root (recursive)."""
    paths = [p for p in glob.glob(os.path.join(root, "**", "*"), recursive=True)
             if p.lower().endswith(IMG_EXTENSIONS)]
    return sorted(paths)


def rgb_to_gray_u8(rgb):
    """uint8 HxWx3 RGB -> HxW gray with OpenCV's fixed-point ITU-R 601 weights."""
    r = rgb[..., 0].astype(np.int32)
    g = rgb[..., 1].astype(np.int32)
    b = rgb[..., 2].astype(np.int32)
    return ((4899 * r + 9617 * g + 1868 * b + 8192) >> 14).astype(np.uint8)


def imread_uint(path, n_channels=3):
    """HxWx1 (gray) or HxWx3 (RGB; gray files replicated) uint8, as utils_image.py:189-201."""
    from PIL import Image
    with Image.open(path) as im:
        if im.mode in ("I;16", "I;16B", "I", "F"):
            raise ValueError(f"{path}: only 8-bit images are supported")
        arr = np.asarray(im.convert("RGB") if im.mode not in ("L", "RGB") else im)
    if n_channels == 1:
        g = arr if arr.ndim == 2 else rgb_to_gray_u8(arr)
        return g[:, :, None]
    if arr.ndim == 2:
        arr = np.repeat(arr[:, :, None], 3, axis=2)
    return np.ascontiguousarray(arr)


def imsave(img, path):
    from PIL import Image
    img = np.squeeze(img)
    Image.fromarray(img.astype(np.uint8)).save(path)


def uint2single(img):
    return np.float32(img / 255.)


def single2uint(img):
    return np.uint8((img.clip(0, 1) * 255.).round())


def single2tensor4(img):
    return torch.from_numpy(np.ascontiguousarray(img)).permute(2, 0, 1).float().unsqueeze(0)


def tensor2uint(img):
    img = img.detach().squeeze().float().clamp(0, 1).cpu().numpy()
    if img.ndim == 3:
        img = np.transpose(img, (1, 2, 0))
    return np.uint8((img * 255.0).round())


def modcrop(img, scale):
    """Crop H and W down to multiples of scale."""
    h, w = img.shape[:2]
    return img[:h - h % scale, :w - w % scale, ...]


def rgb2ycbcr(img, only_y=True):
    """MATLAB rgb2ycbcr (ITU-R BT.601, studio range) for uint8 [0, 255] or float [0, 1] input."""
    in_type = img.dtype
    x = img.astype(np.float64)
    if in_type != np.uint8:
        x = x * 255.
    if only_y:
        out = x @ np.array([65.481, 128.553, 24.966]) / 255.0 + 16.0
    else:
        out = x @ np.array([[65.481, -37.797, 112.0], [128.553, -74.203, -93.786],
                            [24.966, 112.0, -18.214]]) / 255.0 + np.array([16., 128., 128.])
    if in_type == np.uint8:
        out = out.round()
    else:
        out = out / 255.
    return out.astype(in_type)


# ---------------------------------------------------------------------------------------------
# Metrics
# ---------------------------------------------------------------------------------------------
def calculate_psnr(img1, img2, border=0):
    """20 log10(255 / RMSE) over the images with `border` pixels shaved on each side."""
    if img1.shape != img2.shape:
        raise ValueError("Input images must have the same dimensions.")
    h, w = img1.shape[:2]
    a = img1[border:h - border, border:w - border].astype(np.float64)
    b = img2[border:h - border, border:w - border].astype(np.float64)
    mse = np.mean((a - b) ** 2)
    if mse == 0:
        return float("inf")
    return 20 * math.log10(255.0 / math.sqrt(mse))


def gaussian_window(size=11, sigma=1.5):
    """Normalised 1-D Gaussian taps exp(-(i - (size-1)/2)^2 / (2 sigma^2)), i < size."""
    i = np.arange(size, dtype=np.float64) - (size - 1) / 2.0
    g = np.exp(-(i * i) / (2.0 * sigma * sigma))
    return g / g.sum()


def _filter_valid(img, g):
    """Separable correlation with the 2-D window outer(g, g), 'valid' part only."""
    n = g.size
    h, w = img.shape
    rows = sum(g[k] * img[k:h - n + 1 + k, :] for k in range(n))
    return sum(g[k] * rows[:, k:w - n + 1 + k] for k in range(n))


def _ssim_2d(img1, img2):
    c1 = (0.01 * 255) ** 2
    c2 = (0.03 * 255) ** 2
    a = img1.astype(np.float64)
    b = img2.astype(np.float64)
    g = gaussian_window(11, 1.5)
    mu1, mu2 = _filter_valid(a, g), _filter_valid(b, g)
    s11 = _filter_valid(a * a, g) - mu1 * mu1
    s22 = _filter_valid(b * b, g) - mu2 * mu2
    s12 = _filter_valid(a * b, g) - mu1 * mu2
    m = ((2 * mu1 * mu2 + c1) * (2 * s12 + c2)) / ((mu1 * mu1 + mu2 * mu2 + c1) * (s11 + s22 + c2))
    return float(m.mean())


def calculate_ssim(img1, img2, border=0):
    """Mean SSIM (11x11 Gaussian window, sigma 1.5, valid region), averaged over RGB channels."""
    if img1.shape != img2.shape:
        raise ValueError("Input images must have the same dimensions.")
    h, w = img1.shape[:2]
    a = img1[border:h - border, border:w - border]
    b = img2[border:h - border, border:w - border]
    if a.ndim == 2:
        return _ssim_2d(a, b)
    if a.ndim == 3 and a.shape[2] == 3:
        return float(np.mean([_ssim_2d(a[:, :, i], b[:, :, i]) for i in range(3)]))
    if a.ndim == 3 and a.shape[2] == 1:
        return _ssim_2d(a[:, :, 0], b[:, :, 0])
    raise ValueError("Wrong input image dimensions.")


# ---------------------------------------------------------------------------------------------
# Degradations
# ---------------------------------------------------------------------------------------------
def _cubic(x):
    """Keys cubic convolution kernel with a = -0.5 (MATLAB imresize 'bicubic')."""
    ax = np.abs(x)
    ax2, ax3 = ax * ax, ax * ax * ax
    return ((1.5 * ax3 - 2.5 * ax2 + 1.0) * (ax <= 1)
            + (-0.5 * ax3 + 2.5 * ax2 - 4.0 * ax + 2.0) * ((ax > 1) & (ax <= 2)))


def _resize_weights(n_in, n_out, scale, antialias):
    """Per-output-sample source indices (0-based, mirrored into range) and weights of one axis."""
    width = 4.0
    shrink = antialias and scale < 1
    if shrink:
        width = width / scale
    x = np.arange(1, n_out + 1, dtype=np.float64)
    u = x / scale + 0.5 * (1.0 - 1.0 / scale)  # output sample centre in input coordinates (1-based)
    left = np.floor(u - width / 2.0)
    taps = int(math.ceil(width)) + 2
    idx = left[:, None] + np.arange(taps)[None, :]  # 1-based
    d = u[:, None] - idx
    wts = scale * _cubic(d * scale) if shrink else _cubic(d)
    wts = wts / wts.sum(axis=1, keepdims=True)
    keep = np.any(wts != 0, axis=0)  # drop taps that are zero for every output sample
    idx, wts = idx[:, keep], wts[:, keep]
    # symmetric extension (edge sample repeated): ... 2 1 | 1 2 ... n | n n-1 ...
    i0 = idx.astype(np.int64) - 1
    period = 2 * n_in
    m = np.mod(i0, period)
    src = np.where(m < n_in, m, period - 1 - m)
    return src, wts


def imresize_np(img, scale, antialiasing=True):
    """MATLAB-style bicubic resize of an HxW or HxWxC float array by `scale` (output
    ceil(H scale) x ceil(W scale)); rows first, then columns."""
    squeeze = img.ndim == 2
    x = img[:, :, None] if squeeze else img
    h, w, _ = x.shape
    oh, ow = int(math.ceil(h * scale)), int(math.ceil(w * scale))
    src_h, w_h = _resize_weights(h, oh, scale, antialiasing)
    src_w, w_w = _resize_weights(w, ow, scale, antialiasing)
    x64 = x.astype(np.float64)
    t = np.einsum("ok,okc->oc", w_h, x64[src_h].reshape(oh, src_h.shape[1], -1)).reshape(oh, w, -1)
    t = np.einsum("pk,opkc->opc", w_w, t[:, src_w, :])
    out = t.astype(img.dtype)
    return out[:, :, 0] if squeeze else out


def wrap_blur(img, kernel):
    """Circular 2-D convolution of each channel of an HxWxC image with a kh x kw kernel, centred at
    (kh // 2, kw // 2) (scipy.ndimage.convolve with mode='wrap')."""
    from scipy import ndimage
    return ndimage.convolve(img, kernel[..., np.newaxis], mode="wrap")


def downsample(img, sf):
    """Standard s-fold decimation at offset 0: img[0::sf, 0::sf]."""
    return img[0::sf, 0::sf, ...]


# ---------------------------------------------------------------------------------------------
# Command line: the three test scripts' loops
# ---------------------------------------------------------------------------------------------
def _device():
    return torch.device("cuda" if torch.cuda.is_available() else "cpu")


def _model_device(model):
    p = next(model.parameters(), None)
    return p.device if p is not None else _device()


def _load(model, path):
    if path:
        model.load_state_dict(torch.load(path, map_location="cpu", weights_only=True), strict=True)
    model.eval()
    for p in model.parameters():
        p.requires_grad_(False)
    return model.to(_device())


def eval_dncnn(paths, model, noise_level, out_dir=None):
    """Gray denoising (main_test_converse_dncnn.py:110-171): AWGN of noise_level / 255 with
    np.random.seed(0) per image; PSNR / SSIM without a border."""
    res = []
    for p in paths:
        img_h = imread_uint(p, 1)
        img_l = uint2single(img_h)
        np.random.seed(seed=0)
        img_l = img_l + np.random.normal(0, noise_level / 255., img_l.shape)
        with torch.no_grad():
            img_e = tensor2uint(model(single2tensor4(img_l).to(_model_device(model))))
        h = img_h.squeeze()
        res.append((os.path.basename(p), calculate_psnr(img_e, h), calculate_ssim(img_e, h)))
        if out_dir:
            imsave(img_e, os.path.join(out_dir, os.path.basename(p)))
    return res


def eval_srresnet(paths, model, sf, out_dir=None):
    """Bicubic super-resolution (main_test_converse_srresnet.py:115-171): modcrop to sf, bicubic x1/sf,
    PSNR / SSIM on RGB and on Y with a border of sf."""
    res = []
    for p in paths:
        img_h = modcrop(imread_uint(p, 3), sf)
        img_l = imresize_np(uint2single(img_h), 1.0 / sf, True)
        with torch.no_grad():
            img_e = tensor2uint(model(single2tensor4(img_l).to(_model_device(model))))
        psnr, ssim = calculate_psnr(img_e, img_h, sf), calculate_ssim(img_e, img_h, sf)
        ey, hy = rgb2ycbcr(img_e, True), rgb2ycbcr(img_h, True)
        res.append((os.path.basename(p), psnr, ssim, calculate_psnr(ey, hy, sf), calculate_ssim(ey, hy, sf)))
        if out_dir:
            imsave(img_e, os.path.join(out_dir, os.path.splitext(os.path.basename(p))[0] + ".png"))
    return res


def eval_usrnet(paths, model, kernel, sf, noise_level=2.55, out_dir=None):
    """Blind deblurring / SR (main_test_converse_usrnet.py:130-192): modcrop to lcm(sf, 8), wrap blur,
    decimation at offset 0, AWGN of noise_level / 255 with np.random.seed(0); PSNR with a border of
    sf^2.  The model takes only the degraded image (ConverseNet, or ConverseUSRNet via a wrapper
    that supplies the kernel and scale)."""
    res = []
    for p in paths:
        img_h = modcrop(imread_uint(p, 3), int(np.lcm(sf, 8)))
        img_l = downsample(wrap_blur(img_h, kernel), sf)
        img_l = uint2single(img_l)
        np.random.seed(seed=0)
        img_l = img_l + np.random.normal(0, noise_level / 255., img_l.shape)
        with torch.no_grad():
            img_e = tensor2uint(model(single2tensor4(img_l).to(_model_device(model))))
        res.append((os.path.basename(p), calculate_psnr(img_e, img_h, sf * sf)))
        if out_dir:
            imsave(img_e, os.path.join(out_dir, os.path.splitext(os.path.basename(p))[0] + f"_x{sf}.png"))
    return res


def main(argv=None):
    ap = argparse.ArgumentParser(description="Run a Converse model over a folder of images and report PSNR / SSIM.")
    ap.add_argument("task", choices=["dncnn", "srresnet", "usrnet"])
    ap.add_argument("--testset", required=True, help="folder of ground-truth images")
    ap.add_argument("--model-path", default=None, help="state dict (.pth); random init when omitted")
    ap.add_argument("--noise-level", type=float, default=None, help="AWGN level in [0, 255] units")
    ap.add_argument("--sf", type=int, default=None, help="scale factor (srresnet: 4, usrnet: 1)")
    ap.add_argument("--kernel", default=None, help="usrnet: blur kernel (.npy)")
    ap.add_argument("--results", default=None, help="folder for the estimated images")
    args = ap.parse_args(argv)
    paths = get_image_paths(args.testset)
    if not paths:
        raise SystemExit(f"no images under {args.testset}")
    if args.results:
        os.makedirs(args.results, exist_ok=True)
    if args.task == "dncnn":
        from .converse_dncnn import ConverseDnCNN
        model = _load(ConverseDnCNN(in_channels=1, kernel_size=7, num_features=64, padding=6,
                                    padding_mode="circular"), args.model_path)
        res = eval_dncnn(paths, model, 25 if args.noise_level is None else args.noise_level, args.results)
        for name, psnr, ssim in res:
            print(f"{name} - PSNR: {psnr:.2f} dB; SSIM: {ssim:.4f}.")
        print(f"Average PSNR/SSIM - PSNR: {np.mean([r[1] for r in res]):.2f} dB; "
              f"SSIM: {np.mean([r[2] for r in res]):.4f}")
    elif args.task == "srresnet":
        from .converse_srresnet import ConverseMSRResNet
        sf = args.sf or 4
        model = _load(ConverseMSRResNet(in_channels=3, out_channels=3, num_features=64, num_blocks=16, upscale=sf),
                      args.model_path)
        res = eval_srresnet(paths, model, sf, args.results)
        for name, psnr, ssim, psnr_y, ssim_y in res:
            print(f"{name} - PSNR: {psnr:.2f} dB; SSIM: {ssim:.4f}; PSNR_Y: {psnr_y:.2f} dB; SSIM_Y: {ssim_y:.4f}.")
        print(f"Average PSNR/SSIM(RGB) - PSNR: {np.mean([r[1] for r in res]):.2f} dB; "
              f"SSIM: {np.mean([r[2] for r in res]):.4f}")
        print(f"Average PSNR/SSIM(Y) - PSNR: {np.mean([r[3] for r in res]):.2f} dB; "
              f"SSIM: {np.mean([r[4] for r in res]):.4f}")
    else:
        from .converse_usrnet import ConverseNet
        if not args.kernel:
            raise SystemExit("usrnet needs --kernel (a blur kernel .npy, e.g. blur_kernels/kernel_1.npy)")
        kernel = np.load(args.kernel, allow_pickle=False)
        sf = args.sf or 1
        model = _load(ConverseNet(num_iterations=5, in_channels=64, num_blocks=7), args.model_path)
        res = eval_usrnet(paths, model, kernel, sf, 2.55 if args.noise_level is None else args.noise_level,
                          args.results)
        for name, psnr in res:
            print(f"{name} -- x{sf} PSNR: {psnr:.2f}dB")
        print(f"Average PSNR(RGB) x{sf}: {np.mean([r[1] for r in res]):.2f} dB")


if __name__ == "__main__":
    main()
