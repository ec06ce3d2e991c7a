"""Evaluation utilities (conversenet_amd/evaluate.py; reference utils/utils_image.py:189-696 and the
main_test_converse_*.py loops), pinned by closed forms and direct evaluations."""
import math
import os

import numpy as np
import pytest

from conversenet_amd import evaluate as E

REF = "/root/reference"


def test_psnr_closed_form_border_and_identity():
    a = np.zeros((10, 12), np.uint8)
    b = np.ones((10, 12), np.uint8)
    assert E.calculate_psnr(a, b) == pytest.approx(20 * math.log10(255.0))
    c = b.copy()
    c[0, :] = 9  # only in the shaved border
    assert E.calculate_psnr(a, c, border=1) == pytest.approx(20 * math.log10(255.0))
    assert E.calculate_psnr(a, c) < E.calculate_psnr(a, b)
    assert E.calculate_psnr(a, a) == float("inf")
    with pytest.raises(ValueError):
        E.calculate_psnr(a, a[:5])


def test_gaussian_window_is_opencv_gaussian():
    g = E.gaussian_window(11, 1.5)
    assert g.sum() == pytest.approx(1.0, abs=1e-15)
    np.testing.assert_allclose(g, g[::-1], atol=0)
    # consecutive taps: exp(-(i^2 - (i-1)^2) / (2 sigma^2))
    for i in range(1, 6):
        assert g[5 + i] / g[5 + i - 1] == pytest.approx(math.exp(-(2 * i - 1) / 4.5))


def _ssim_direct(a, b):
    """SSIM by its definition: every 11x11 window weighted by the Gaussian, summed directly."""
    c1, c2 = (0.01 * 255) ** 2, (0.03 * 255) ** 2
    g = E.gaussian_window(11, 1.5)
    w = np.outer(g, g)
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    vals = []
    for i in range(a.shape[0] - 10):
        for j in range(a.shape[1] - 10):
            pa, pb = a[i:i + 11, j:j + 11], b[i:i + 11, j:j + 11]
            m1, m2 = (w * pa).sum(), (w * pb).sum()
            v1 = (w * pa * pa).sum() - m1 * m1
            v2 = (w * pb * pb).sum() - m2 * m2
            cv = (w * pa * pb).sum() - m1 * m2
            vals.append(((2 * m1 * m2 + c1) * (2 * cv + c2)) / ((m1 * m1 + m2 * m2 + c1) * (v1 + v2 + c2)))
    return float(np.mean(vals))


def test_ssim_matches_direct_definition_and_special_cases():
    rng = np.random.default_rng(0)
    a = rng.integers(0, 256, (20, 23)).astype(np.uint8)
    b = np.clip(a.astype(int) + rng.integers(-30, 31, a.shape), 0, 255).astype(np.uint8)
    assert E.calculate_ssim(a, b) == pytest.approx(_ssim_direct(a, b), abs=1e-12)
    assert E.calculate_ssim(a, a) == pytest.approx(1.0, abs=1e-12)
    # constant images: sigmas vanish, SSIM = (2 c1 c2 + C1) / (c1^2 + c2^2 + C1)
    k1 = (0.01 * 255) ** 2
    s = E.calculate_ssim(np.full((16, 16), 40, np.uint8), np.full((16, 16), 90, np.uint8))
    assert s == pytest.approx((2 * 40 * 90 + k1) / (40 ** 2 + 90 ** 2 + k1))
    # RGB: mean over channels; HxWx1 squeezed; border shaving
    rgb_a = np.stack([a, b, a], 2)
    rgb_b = np.stack([b, b, a], 2)
    assert E.calculate_ssim(rgb_a, rgb_b) == pytest.approx((_ssim_direct(a, b) + 2.0) / 3, abs=1e-12)
    assert E.calculate_ssim(a[:, :, None], b[:, :, None]) == pytest.approx(E.calculate_ssim(a, b))
    assert E.calculate_ssim(a, b, border=2) == pytest.approx(_ssim_direct(a[2:-2, 2:-2], b[2:-2, 2:-2]), abs=1e-12)


def test_rgb2ycbcr_studio_range():
    white = np.full((1, 1, 3), 255, np.uint8)
    black = np.zeros((1, 1, 3), np.uint8)
    assert E.rgb2ycbcr(white)[0, 0] == 235 and E.rgb2ycbcr(black)[0, 0] == 16
    red = np.array([[[255, 0, 0]]], np.uint8)
    assert E.rgb2ycbcr(red)[0, 0] == round(65.481 + 16)
    full = E.rgb2ycbcr(white, only_y=False)[0, 0]
    np.testing.assert_array_equal(full, [235, 128, 128])
    f = E.rgb2ycbcr(np.ones((1, 1, 3), np.float32))
    assert f[0, 0] == pytest.approx(235 / 255, abs=1e-6)


def test_conversions_and_modcrop():
    img = np.arange(0, 256, dtype=np.uint8).reshape(16, 16)
    assert np.array_equal(E.single2uint(E.uint2single(img)), img)
    t = E.single2tensor4(E.uint2single(img)[:, :, None])
    assert t.shape == (1, 1, 16, 16)
    assert np.array_equal(E.tensor2uint(t), img)
    assert E.modcrop(np.zeros((17, 23, 3)), 4).shape == (16, 20, 3)


def test_imread_uint_and_gray_weights(tmp_path):
    from PIL import Image
    rng = np.random.default_rng(1)
    rgb = rng.integers(0, 256, (9, 7, 3)).astype(np.uint8)
    p = str(tmp_path / "x.png")
    Image.fromarray(rgb).save(p)
    assert np.array_equal(E.imread_uint(p, 3), rgb)
    g = E.imread_uint(p, 1)[:, :, 0]
    ref = np.floor(rgb.astype(np.float64) @ np.array([0.299, 0.587, 0.114]) + 0.5)
    assert np.abs(g.astype(int) - ref).max() <= 1  # fixed-point rounding of the 601 weights
    assert E.rgb_to_gray_u8(np.array([[[255, 0, 0]]], np.uint8))[0, 0] == 76  # 0.299 * 255 = 76.2
    gray = rng.integers(0, 256, (5, 6)).astype(np.uint8)
    Image.fromarray(gray).save(p)
    assert np.array_equal(E.imread_uint(p, 1)[:, :, 0], gray)
    assert np.array_equal(E.imread_uint(p, 3), np.repeat(gray[:, :, None], 3, 2))
    E.imsave(rgb, p)
    assert np.array_equal(E.imread_uint(p, 3), rgb)


@pytest.mark.parametrize("scale", [0.5, 0.25, 2.0, 3.0])
def test_imresize_sampling_positions_and_partition_of_unity(scale):
    h, w = 24, 36
    # constant in -> constant out (weights of every output sample sum to 1)
    c = np.full((h, w), 0.37)
    out = E.imresize_np(c, scale)
    assert out.shape == (math.ceil(h * scale), math.ceil(w * scale))
    np.testing.assert_allclose(out, 0.37, atol=1e-12)
    # a linear ramp is reproduced exactly away from the symmetric borders, at the output sample
    # centres u = x / scale + (1 - 1 / scale) / 2 (1-based): pins the index mapping
    ramp = np.tile(np.arange(1, w + 1, dtype=np.float64), (h, 1))
    r = E.imresize_np(ramp, scale)
    x = np.arange(1, r.shape[1] + 1)
    u = x / scale + 0.5 * (1 - 1 / scale)
    half = 2.0 / min(scale, 1.0) + 2
    inner = (u - half >= 1) & (u + half <= w)
    np.testing.assert_allclose(r[:, inner], np.broadcast_to(u[inner], r[:, inner].shape), atol=1e-9)
    assert inner.sum() >= 2


def test_imresize_identity_and_symmetry():
    rng = np.random.default_rng(2)
    img = rng.random((10, 14, 3))
    np.testing.assert_allclose(E.imresize_np(img, 1.0), img, atol=1e-12)
    sym = img + img[:, ::-1]  # left-right symmetric input -> symmetric output
    out = E.imresize_np(sym, 0.5)
    np.testing.assert_allclose(out, out[:, ::-1], atol=1e-12)


def test_wrap_blur_is_centred_circular_convolution():
    rng = np.random.default_rng(3)
    img = rng.random((12, 10, 2))
    k = rng.random((5, 5))
    k /= k.sum()
    got = E.wrap_blur(img, k)
    # circular convolution with the kernel's centre (2, 2) at the origin, by FFT
    kp = np.zeros((12, 10))
    kp[:5, :5] = k
    kp = np.roll(kp, (-2, -2), axis=(0, 1))
    want = np.real(np.fft.ifft2(np.fft.fft2(img, axes=(0, 1)) * np.fft.fft2(kp)[:, :, None], axes=(0, 1)))
    np.testing.assert_allclose(got, want, atol=1e-12)
    delta = np.zeros((3, 3))
    delta[1, 1] = 1
    np.testing.assert_allclose(E.wrap_blur(img, delta), img, atol=0)
    assert E.downsample(img, 3).shape == (4, 4, 2)


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "model_zoo")), reason="reference checkpoints absent")
def test_pretrained_dncnn_denoises_reference_image(tmp_path, capsys):
    """End to end on the CPU path: the shipped Converse-DnCNN checkpoint on a 96x96 gray crop of the
    reference's utils/test.png with AWGN sigma 25 (np.random.seed(0)) must beat the noisy input's
    PSNR by a wide margin; the command line runs the same loop."""
    from PIL import Image
    img = E.imread_uint(os.path.join(REF, "utils", "test.png"), 1)[400:496, 400:496, 0]
    d = tmp_path / "set"
    d.mkdir()
    Image.fromarray(img).save(str(d / "crop.png"))
    from conversenet_amd.converse_dncnn import ConverseDnCNN
    model = E._load(ConverseDnCNN(), os.path.join(REF, "model_zoo", "converse_dncnn.pth"))
    (name, psnr, ssim), = E.eval_dncnn(E.get_image_paths(str(d)), model, 25)
    np.random.seed(0)
    noisy = E.single2uint(E.uint2single(img[:, :, None]) + np.random.normal(0, 25 / 255., (96, 96, 1)))[:, :, 0]
    assert psnr > E.calculate_psnr(noisy, img) + 5.0 and ssim > E.calculate_ssim(noisy, img)
    E.main(["dncnn", "--testset", str(d), "--model-path", os.path.join(REF, "model_zoo", "converse_dncnn.pth")])
    assert f"PSNR: {psnr:.2f} dB" in capsys.readouterr().out
