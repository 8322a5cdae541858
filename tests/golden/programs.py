"""The Anvil programs behind the golden fixtures (written for this repository).

Each entry: name, source, optional consts (the `--set` overrides), seed, and
  interp: True    -> the reference interpreter runs it and its vectors are kept,
  keep: [...]     -> buffer names whose final contents are kept,
  function: {...} -> lower one function with pyapi.lower for these argument shapes,
  stdin: "..."    -> what `input` reads.
The configurations C1-C5 are the workloads named in BASELINE.json; the rest restate the cases of
the reference's CUDA backend tests (tests/test_cuda.py:26-159) as programs of their own, and the
run-time calls (data files, checkpoints, input, nonzero) with data files from make_data.py.
"""

# ----------------------------------------------------------------------------- C1: MLP 784-128-10, SGD

C1 = """
const N = 60000
const NT = 10000
const EPOCHS = 1
const BATCH = 64

kx: i32[N, 784] ~ randint(0, 256)
X = f32(kx) / 255
labels: i32[N] ~ randint(0, 10)
kt: i32[NT, 784] ~ randint(0, 256)
X_test = f32(kt) / 255
test_labels: i32[NT] ~ randint(0, 10)

model MLP:
    l1 = Linear(784, 128)
    l2 = Linear(128, 10)
    fn forward(x: [n, 784]) -> [n, 10] = x |> l1 |> relu |> l2

net = MLP()

for epoch in range(EPOCHS):
    for x, y in batches(X, labels, size=BATCH, shuffle=true):
        loss = cross_entropy(net(x), y)
        minimize loss with sgd(lr=0.1)
    acc = accuracy(net(X_test), test_labels)
    print("epoch {epoch + 1}   loss {loss:.4f}   test accuracy {acc:.4f}")
"""

# ----------------------------------------------------------------------------- C2: MLP 784-1024-1024-10, Adam

C2 = """
const N = 65536
const H = 1024
const BATCH = 256
const STEPS = 500
const EPOCHS = 2

X: [N, 784] ~ uniform(0, 1)
labels: i32[N] ~ randint(0, 10)

seed(1)
model WideMLP:
    l1 = Linear(784, H)
    l2 = Linear(H, H)
    l3 = Linear(H, 10)
    fn forward(x) = x |> l1 |> relu |> l2 |> relu |> l3

net = WideMLP()

step = 0
for epoch in range(EPOCHS):
    for x, y in batches(X, labels, size=BATCH, shuffle=true):
        if step >= STEPS:
            break
        loss = cross_entropy(net(x), y)
        minimize loss with adam(lr=1e-3)
        step += 1
        if step == 1:
            print("step 1 loss {loss:.6e}")
print("steps {step}   loss {loss:.4f}")
"""

# ----------------------------------------------------------------------------- C3: standalone functions

C3_SOFTMAX = """
fn rows_softmax(x: [n, d]) = softmax(x)
"""

C3_LAYERNORM = """
fn norm(x: [n, d], g: [d], b: [d]) = layer_norm(x) * g + b
"""

C3_LINEAR = """
fn linear(x: [n, k], W: [o, k], b: [o]):
    y[i, j] = sum W[j, c] * x[i, c] + b[j]
    return y
"""

C3_BMM = """
fn bmm(a: [b, m, k], w: [b, k, n]):
    y[t, i, j] = sum a[t, i, c] * w[t, c, j]
    return y
"""

C3_ATTENTION = """
fn attention(q: [b, t, d], k: [b, t, d], v: [b, t, d]):
    s[n, i, j] = sum q[n, i, c] * k[n, j, c] / sqrt(d)
    return softmax(s) @ v
"""

# ----------------------------------------------------------------------------- C4: char transformer

C4 = """
const STEPS = 200
const BATCH = 16
const T = 64
const D = 256
const HEADS = 4
const DH = D // HEADS
const V = 96
const LAYERS = 4

seed(3)

model Layer:
    param Wqkv: [D, 3 * D] ~ normal(0, sqrt(1 / D))
    param Wout: [D, D] ~ normal(0, sqrt(0.5 / D))
    ff_in = Linear(D, 4 * D)
    ff_out = Linear(4 * D, D)
    fn forward(z):
        qkv = (layer_norm(z) @ Wqkv).reshape(-1, T, 3, HEADS, DH)
        score[n, h, t, u] = sum qkv[n, t, 0, h, c] * qkv[n, u, 1, h, c] / sqrt(DH) - 1e9 * f32(u > t)
        w = softmax(score)
        mix[n, t, h, c] = sum w[n, h, t, u] * qkv[n, u, 2, h, c]
        z = z + mix.reshape(-1, T, D) @ Wout
        return z + ff_out(gelu(ff_in(layer_norm(z))))

model CharModel:
    param tok: [V, D] ~ normal(0, 0.5)
    param pos: [T, D] ~ normal(0, 0.1)
    layers = [Layer() for n in range(LAYERS)]
    head = Linear(D, V)
    fn forward(codes):
        z[n, t, d] = tok[codes[n, t], d] + pos[t, d]
        static for layer in layers:
            z = layer(z)
        return head(layer_norm(z))

net = CharModel()

for step in range(STEPS):
    text: i32[BATCH, T + 1] ~ randint(0, V)
    logits = net(text[:, 0:T])
    loss = cross_entropy(logits.reshape(BATCH * T, V), text[:, 1:T + 1].reshape(BATCH * T))
    minimize loss over net with adam(lr=1e-3)
    if step == 0:
        print("step 1 loss {loss:.6e}")
print("loss {loss:.4f}")
"""

# ----------------------------------------------------------------------------- C5: small CNN

C5 = """
const STEPS = 300
const NB = 128
const C1 = 32
const C2 = 64
const HID = 128

seed(4)
X: [NB, 1, 28, 28] ~ uniform(0, 1)
Y: i32[NB] ~ randint(0, 10)

model Net:
    c1 = Conv2d(1, C1, 3)
    c2 = Conv2d(C1, C2, 3)
    fc1 = Linear(C2 * 12 * 12, HID)
    fc2 = Linear(HID, 10)
    fn forward(x) = x |> c1 |> relu |> c2 |> relu |> max_pool2d |> flatten(1) |> fc1 |> relu |> fc2

net = Net()

for step in range(STEPS):
    loss = cross_entropy(net(X), Y)
    minimize loss with sgd(lr=0.05)
    if step == 0:
        print("step 1 loss {loss:.6e}")
print("loss {loss:.4f}")
"""

# ----------------------------------------------------------------------------- test programs

CHECK_NAN = "x: [4, 3] ~ normal(0, 1)\nw = exp(x)\ny = log(x - 0.5) * w\nprint(sum(y))\n"

CHECK_INF = "x: [4, 3] ~ normal(0, 1)\nz = log(x * 0)\nr = z - z\nprint(sum(r))\n"

CHECK_HEALTHY = """
x: [64, 8] ~ normal(0, 1)
y: [64] ~ normal(0, 1)
param w: [8] ~ normal(0, 1)
for step in range(20):
    loss = mean((x @ w - y) ** 2)
    minimize loss with adam(lr=0.01)
print(loss)
"""

GREET = """
v = [0.5, -1.5, 2.0, 4.0]
M = [[2.0, 1.0, 0.0, -1.0],
     [0.0, 3.0, 1.0, 1.0],
     [1.0, 1.0, 1.0, 1.0]]
r[a] = sum M[a, b] * v[b]
print("r = {r}")
gap[a, b] = v[a] - v[b]
print(gap)
print("logsm {log_softmax(v)} min {min(v)} total {sum(v):.2f}")
u: [3, 2] ~ uniform(-1, 1)
print("u = {u}")
param p: [4]
obj = sum((p * v - 1.0) ** 2)
dp = grad(obj, p)
print("dp {dp}")
"""

LOGREG = """
m = 800
F: [m, 4] ~ normal(0, 1)
z = F @ [1.5, -0.5, 2.0, 0.25] - 0.3
lab = f32(z > 0)

param w: [4]
param c: f32

for it in range(80):
    prob = sigmoid(F @ w + c)
    loss = -mean(lab * log(prob + 1e-6) + (1 - lab) * log(1 - prob + 1e-6))
    minimize loss with sgd(lr=0.5)
    if it % 16 == 0:
        print("iter {it:3d}   loss {loss:.5f}")

print("w = {w}   c = {c:.3f}")
"""

ATTENTION_FIT = """
NB = 4
L = 12
E = 16
K = 8

fn head(z: [b, t, e], A: [e, k], B: [e, k], C: [e, k], O: [k, e]) -> [b, t, e]:
    qq = z @ A
    kk = z @ B
    vv = z @ C
    logit[n, t, u] = sum qq[n, t, c] * kk[n, u, c] * 0.35355339
    att = softmax(logit)
    ctx[n, t, c] = sum att[n, t, u] * vv[n, u, c]
    return ctx @ O

RA: [E, K] ~ normal(0, 0.3)
RB: [E, K] ~ normal(0, 0.3)
RC: [E, K] ~ normal(0, 0.3)
RO: [K, E] ~ normal(0, 0.3)

param A: [E, K] ~ normal(0, 0.1)
param B: [E, K] ~ normal(0, 0.1)
param C: [E, K] ~ normal(0, 0.1)
param O: [K, E] ~ normal(0, 0.1)

for step in range(1, 49):
    z: [NB, L, E] ~ normal(0, 1)
    loss = mse(head(z, A, B, C, O), head(z, RA, RB, RC, RO))
    minimize loss with adam(lr=0.02)
    if step % 12 == 0:
        print("step {step:3d}   loss {loss:.5f}")
"""

SPLIT = """
x: [300000] ~ normal(0, 1)
print("sum {sum(x):.2f}  max {max(x):.4f}  min {min(x):.4f}  mean {mean(x):.5f}")
W: [3, 50000] ~ uniform(-1, 1)
y: [50000] ~ normal(0, 1)
v[i] = sum W[i, j] * y[j]
print(v)
print(argmax(x))
print(argmin(x))
R = rand(3, 50000)
noisy[i] = sum W[i, j] * R[i, j]
print(noisy)
"""

SCATTER = """
labels: i32[1000] ~ randint(0, 10)
counts: i32[10] = 0
counts[labels[i]] += 1
print(counts)
E: [10, 4] ~ normal(0, 1)
rows[i, d] = E[labels[i], d]
print(rows[0:5])
hist: [10] = 0.0
hist[labels[i]] += 0.5
print(hist)
"""

BOUNDS = """
x = arange(10)
for i in range(12):
    s = x[i]
    print(s)
"""

GATHER_OOB = """
idx: i32[4] = [0, 1, 7, 2]
E: [5, 3] ~ normal(0, 1)
r[i, d] = E[idx[i], d]
print(r)
"""

ASSERT_FAIL = """
x = sum(rand(3)) + 3
assert x < 2, "x is too big"
print("unreachable")
"""

SAVE_LOAD = """
param W: [3, 4] ~ normal(0, 1)
loaded = load(W, "CKPT")
if loaded == 0:
    save(W, "CKPT")
print("loaded {loaded} sum {sum(W):.4f}")
"""

INTEGERS = """
a: i32[12] = [-7, -6, -5, -1, 0, 1, 5, 6, 7, 2147483647, -2147483647, 13]
b: i32[12] = [2, -4, 3, 5, 3, -2, 0, 4, -3, 1, 2, -5]
print(a // b)
print(a % b)
print(a + b)
print(a * b)
fa = f32(a) / 4
print(fa // 1.5)
print(fa % -1.5)
print(i32(fa))
print(round(fa))
print(floor(fa))
print(ceil(fa))
print(sign(fa))
print(abs(a))
print(max(fa, 0.5))
print(min(a, 3))
v = [1.5, -2.25, 0.0, 3.75]
print(exp(v))
print(log(abs(v) + 1))
print(sqrt(abs(v)))
print(tanh(v))
print(sigmoid(v))
print(sin(v))
print(cos(v))
print(v ** 2)
print(f32(v > 0) + f32(v <= 0) * 2)
print(argmax(v))
print(prod(v + 3))
"""

FORMATS = """
big: [40, 30] ~ normal(0, 1000)
print(big)
small: [3, 4] ~ uniform(0, 0.0001)
print(small)
i3: i32[2, 3, 4] ~ randint(-50, 50)
print(i3)
long: i32[2000] ~ randint(0, 100)
print(long)
z = 0.0
print("zero {z} int {i3[1, 2, 3]} f {z:.2f}")
"""

CONTROL = """
total = 0
k = 0
while k < 10:
    k += 1
    if k % 3 == 0:
        continue
    total += k
    if total > 20:
        break
print("k {k} total {total}")
acc = 0.0
for i in range(5):
    for j in range(i, 5):
        acc += f32(i * j)
print("acc {acc}")
"""

PRODUCTS = """
x: [6, 40] ~ uniform(0.9, 1.1)
p[i] = prod x[i, j]
print(p)
mx[i] = max x[i, j]
mn[i] = min x[i, k]
print(mx - mn)
a[i] = argmax x[i, j]
print(a)
"""

MNIST_LIKE = """
const N = 2048
const NT = 512
const EPOCHS = 2

kx: i32[N, 784] ~ randint(0, 256)
X = f32(kx) / 255
labels: i32[N] ~ randint(0, 10)
kt: i32[NT, 784] ~ randint(0, 256)
X_test = f32(kt) / 255
test_labels: i32[NT] ~ randint(0, 10)

model MLP:
    l1 = Linear(784, 128)
    l2 = Linear(128, 10)
    fn forward(x: [n, 784]) -> [n, 10] = x |> l1 |> relu |> l2

net = MLP()

for epoch in range(EPOCHS):
    for x, y in batches(X, labels, size=64, shuffle=true):
        loss = cross_entropy(net(x), y)
        minimize loss with sgd(lr=0.1)
    acc = accuracy(net(X_test), test_labels)
    print("epoch {epoch + 1}   loss {loss:.4f}   test accuracy {acc:.4f}")
"""

FILES = """
t = csv("../data/table.csv")
print(t)
print("sum {sum(t):.4f}")
note = bytes("../data/note.txt")
print(note)
tiles = idx("../data/tiles-idx3-ubyte.gz")
print(tiles)
marks: i32[6] = idx("../data/marks-idx1-ubyte")
print(marks)
print(npy("../data/k_f4.npy"))
print(npy("../data/k_f8.npy"))
print(npy("../data/k_f2.npy"))
print(npy("../data/k_i4.npy"))
print(npy("../data/k_i8.npy"))
print(npy("../data/k_u1.npy"))
print(npy("../data/k_i1.npy"))
print(npy("../data/k_u2.npy"))
print(npy("../data/k_i2.npy"))
print(npy("../data/k_b1.npy"))
w = safetensors("../data/layer.safetensors", "layer.w")
print(w)
print(safetensors("../data/layer.safetensors", "layer.half"))
print(safetensors("../data/layer.safetensors", "layer.ids"))
save_npy(w * 2, "OUT_w2.npy")
save_npy(marks + 1, "OUT_marks.npy")
"""

PICKS = """
v: i32[20] ~ randint(0, 3)
print(v)
grid: [3, 5] ~ uniform(-1, 1)
print(grid)
r, c = nonzero(grid > 0.25, size=6, fill_value=-9)
print(r)
print(c)
q, s = nonzero(v.reshape(4, 5) == 2, size=12)
print(q)
print(s)
total = 0.0
for turn in range(20):
    x = input("value? ")
    if x != x:
        print("(no number)")
        continue
    total += x
    print("total {total:.3f}")
"""

PICKS_STDIN = "3\nabc 4.5e1 x\n0x1F\n-.25\nnothing here\n+-2e-1 tail\n1e\n7."

CELL = """
model Cell:
    param gate: [3, 4] ~ uniform(-1, 1)
    param bias: [4] ~ uniform(0, 0.5)

model Pair:
    left = Cell()
    right = Cell()
    param scale: [2] ~ uniform(1, 2)
"""

CKPT_WRITE = CELL + """
seed(21)
net = Pair()
print("gate sum {sum(net.left.gate):.6f}   scale {net.scale}")
save(net, "OUT_pair.ckpt")
"""

CKPT_READ = CELL + """
model Swapped:
    param gate: [4, 3] ~ uniform(-1, 1)
    param bias: [4] ~ uniform(0, 0.5)

seed(22)
net = Pair()
got = load(net, "../data/pair.ckpt")
print("loaded {got}")
print(net.left.gate)
print(net.right.bias)
print(net.scale)
other = Swapped()
before = sum(other.gate)
miss = load(other, "../data/pair.ckpt")
print("mismatched {miss} unchanged {sum(other.gate) == before}")
none = load(net, "../data/no-such.ckpt")
print("absent {none}")
"""

SERIAL = """
order: i32[10] = [2, 0, 2, 1, 3, 0, 2, 1, 1, 3]
vals: [10] ~ uniform(0, 1)
slots: [4] = 0.0
slots[order] = vals
print(slots)
pick: i32[6] = [5, 5, 0, 5, 2, 0]
dst: i32[6] = 0
dst[pick] = pick * 10 + arange(6)
print(dst)
"""

BOARD = """
cells: i32[3, 6] ~ randint(0, 6)
show(cells, ".#o*")
print(cells)
"""

DRAWS = """
seed(5)
u: [3, 4] ~ uniform(-2, 2)
k: i32[40] ~ randint(-5, 17)
b: [10] ~ bernoulli(0.6)
m: i32[2, 3] ~ randint(0, 1000)
g: [5] ~ uniform(0, 1)
print(i32(u * 4194304.0))
print(i32(g * 16777216.0))
print(u)
print(k)
print(b)
print(m)
"""

# argmax / argmin as np.argmax / np.argmin decide (interp.py:478-481): the first of equal extremes,
# a nan before every number (the first nan), rows of -inf and of zeros; one lane per row (20), a
# wavefront per row (64), a workgroup per row (256, 5000, 8192), whole tensors, and whole tensors
# past the interpreter's chunk of 2^22 elements, whose chunk picks meet by its own rule (a later
# chunk holding a nan is passed over: gA's 9.0 never wins)
ARGPICK = """
const BIG = 4198400
neg: [2] = -1.0
bad = sqrt(neg)
zero: [2] = 0.0
ninf = log(zero)
s20[i, j] = f32((j * 7 + i) % 5) where i < 300, j < 20
n20[i, j] = (bad[0] if (j == i % 23 and i % 3 == 0) else (ninf[0] if i % 7 == 1 else s20[i, j]))
a20[i] = argmax n20[i, j]
b20[i] = argmin n20[i, j]
print(a20)
print(b20)
t64[i, j] = f32((j * 5 + i * 3) % 8) where i < 256, j < 64
n64[i, j] = (bad[0] if j == (i * 13) % 80 else (ninf[0] if i % 11 == 5 else t64[i, j]))
a64[i] = argmax n64[i, j]
b64[i] = argmin n64[i, j]
print(a64)
print(b64)
t256[i, j] = f32((j * 37 + i) % 61) where i < 6, j < 256
n256[i, j] = (bad[0] if (i == 2 and j == 200) or (i == 4 and (j == 3 or j == 250)) else t256[i, j])
rz[i, j] = max(t256[i, j] - 100.0, 0.0)
a256[i] = argmax n256[i, j]
b256[i] = argmin n256[i, j]
c256[i] = argmax rz[i, j]
d256[i] = argmin rz[i, j]
print(a256)
print(b256)
print(c256)
print(d256)
t5k[i, j] = f32((j * 13 + i * 7) % 97) where i < 3, j < 5000
n5k[i, j] = (bad[0] if i == 1 and j == 4700 else t5k[i, j])
a5k[i] = argmax n5k[i, j]
b5k[i] = argmin n5k[i, j]
print(a5k)
print(b5k)
t8k[i, j] = f32((j * 29 + i) % 101) where i < 2, j < 8192
n8k[i, j] = (bad[0] if i == 0 and (j == 8000 or j == 8191) else t8k[i, j])
a8k[i] = argmax n8k[i, j]
b8k[i] = argmin n8k[i, j]
print(a8k)
print(b8k)
w[j] = f32((j * 7919) % 1000) where j < 300000
wn[j] = (bad[0] if j == 250001 else w[j])
print(argmax(w))
print(argmin(w))
print(argmax(wn))
print(argmin(wn))
g[j] = f32(j % 5) where j < BIG
gA[j] = (bad[0] if j == 4194400 else (9.0 if j == 4194500 else g[j]))
gB[j] = (bad[0] if j == 3000000 or j == 10 else g[j])
gC[j] = (9.0 if j == 4194310 else g[j])
gD[j] = (-3.0 if j == 4194305 or j == 17 else g[j])
print(argmax(gA))
print(argmin(gA))
print(argmax(gB))
print(argmax(gC))
print(argmin(gD))
"""

C4_MID = {"STEPS": 2, "BATCH": 4, "T": 32, "D": 64, "HEADS": 2, "LAYERS": 1}
C1_KEEP = ["net.l1.W", "net.l1.b", "net.l2.W", "net.l2.b", "perm"]
C2_KEEP = ["net.l1.W", "net.l1.b", "net.l2.W", "net.l2.b", "net.l3.W", "net.l3.b", "perm"]

PROGRAMS = [
    # the workloads at the sizes BASELINE.json names (IR only: the interpreter would take hours)
    {"name": "c1_mlp", "source": C1},
    # C1 and C2 whole, as BASELINE.json states them, through the reference interpreter: the printed
    # loss and accuracy and the last layer's trained weights
    {"name": "c1_full", "source": C1, "interp": True, "keep": ["net.l2.W", "net.l2.b"]},
    {"name": "c2_full", "source": C2, "interp": True, "keep": ["net.l3.W", "net.l3.b"]},
    {"name": "c4_full2", "source": C4, "consts": {"STEPS": 2}, "interp": True,
     "keep": ["net.layers.0.Wqkv", "net.layers.3.ff_in.W", "net.head.W", "net.head.b"]},
    {"name": "c5_full3", "source": C5, "consts": {"STEPS": 3}, "interp": True,
     "keep": ["net.c1.W", "net.c1.b", "net.c2.W", "net.c2.b", "net.fc2.W"]},
    {"name": "c2_full10", "source": C2, "consts": {"STEPS": 10}, "interp": True,
     "keep": ["net.l1.b", "net.l2.b", "net.l3.W", "net.l3.b"]},
    {"name": "c2_wide_mlp", "source": C2},
    {"name": "c4_transformer", "source": C4},
    {"name": "c4_transformer_t256", "source": C4, "consts": {"T": 256}},
    {"name": "c5_cnn", "source": C5},
    {"name": "c3_softmax", "source": C3_SOFTMAX,
     "function": {"name": "rows_softmax", "args": [([8192, 4096], "f32")]}},
    {"name": "c3_layernorm", "source": C3_LAYERNORM,
     "function": {"name": "norm", "args": [([8192, 1024], "f32"), ([1024], "f32"), ([1024], "f32")]}},
    {"name": "c3_linear", "source": C3_LINEAR,
     "function": {"name": "linear", "args": [([8192, 4096], "f32"), ([4096, 4096], "f32"), ([4096], "f32")]}},
    # products whose shapes take one wavefront of 2 x 2 MFMA tiles (IR only; the GPU tests check them
    # against float64 closed forms)
    {"name": "c3_linear_mid", "source": C3_LINEAR,
     "function": {"name": "linear", "args": [([4096, 256], "f32"), ([1024, 256], "f32"), ([1024], "f32")]}},
    # C2's layer shape as x·Wᵀ (both operands contiguous in k, as in C2's input gradient)
    {"name": "c3_linear_b256", "source": C3_LINEAR,
     "function": {"name": "linear", "args": [([256, 1024], "f32"), ([1024, 1024], "f32"), ([1024], "f32")]}},
    {"name": "c3_bmm", "source": C3_BMM,
     "function": {"name": "bmm", "args": [([64, 256, 64], "f32"), ([64, 64, 256], "f32")]}},
    {"name": "c3_attention", "source": C3_ATTENTION,
     "function": {"name": "attention", "args": [([4, 2048, 128], "f32")] * 3}},
    # the same workloads at sizes the interpreter finishes in seconds (IR + vectors)
    {"name": "c1_small", "source": C1, "consts": {"N": 640, "NT": 256}, "interp": True, "keep": C1_KEEP},
    {"name": "c2_small", "source": C2, "consts": {"N": 1024, "H": 96, "BATCH": 32, "STEPS": 40},
     "interp": True, "keep": C2_KEEP},
    {"name": "c2_steps100", "source": C2, "consts": {"N": 2048, "H": 64, "BATCH": 32, "STEPS": 100},
     "interp": True, "keep": C2_KEEP},
    {"name": "c4_small", "source": C4,
     "consts": {"STEPS": 3, "BATCH": 2, "T": 8, "D": 32, "HEADS": 2, "LAYERS": 2}, "interp": True},
    # C4 at a size where its products are matrix-core products, the input gradients that add
    # q, k and v's contributions (`+=`) among them
    {"name": "c4_mid", "source": C4,
     "consts": {"STEPS": 2, "BATCH": 4, "T": 32, "D": 64, "HEADS": 2, "LAYERS": 1}, "interp": True,
     "keep": ["net.tok", "net.layers.0.Wqkv", "net.layers.0.ff_in.W", "net.head.W"]},
    {"name": "c5_small", "source": C5, "consts": {"STEPS": 3, "NB": 4, "C1": 4, "C2": 8, "HID": 16},
     "interp": True},
    # C5 at a size where the convolution's weight gradient is a product with K over the batch and
    # the positions, split across workgroups, and fc1 (32 x 32, K = 9216) splits K as well
    {"name": "c5_mid", "source": C5, "consts": {"STEPS": 2, "NB": 32, "C1": 8, "C2": 32, "HID": 32},
     "interp": True, "keep": ["net.c1.W", "net.c2.W", "net.fc1.W", "net.fc2.W"]},
    {"name": "c3_softmax_small", "source": C3_SOFTMAX, "interp": True,
     "function": {"name": "rows_softmax", "args": [([64, 300], "f32")]}},
    {"name": "c3_layernorm_small", "source": C3_LAYERNORM, "interp": True,
     "function": {"name": "norm", "args": [([48, 200], "f32"), ([200], "f32"), ([200], "f32")]}},
    {"name": "c3_linear_small", "source": C3_LINEAR, "interp": True,
     "function": {"name": "linear", "args": [([96, 80], "f32"), ([72, 80], "f32"), ([72], "f32")]}},
    # a tall product (2048 x 128 outputs: 64 x 4 tiles), launched in the XCD-aware tile order
    {"name": "c3_linear_tall", "source": C3_LINEAR, "interp": True,
     "function": {"name": "linear", "args": [([2048, 64], "f32"), ([128, 64], "f32"), ([128], "f32")]}},
    {"name": "c3_attention_small", "source": C3_ATTENTION, "interp": True,
     "function": {"name": "attention", "args": [([2, 64, 32], "f32")] * 3}},
    # the same function at half the keys and head size: a second, smaller compilation
    {"name": "c3_attention_tiny", "source": C3_ATTENTION, "interp": True,
     "function": {"name": "attention", "args": [([2, 32, 16], "f32")] * 3}},
    # shapes the one-kernel attention takes (head size 64 and 128, keys a multiple of 128)
    {"name": "c3_attention_d64", "source": C3_ATTENTION, "interp": True,
     "function": {"name": "attention", "args": [([2, 128, 64], "f32")] * 3}},
    {"name": "c3_attention_d128", "source": C3_ATTENTION, "interp": True,
     "function": {"name": "attention", "args": [([2, 256, 128], "f32")] * 3}},
    # --check (the reference's tests/test_native.py:292-320): unoptimized, one kernel per operation
    {"name": "check_nan", "source": CHECK_NAN, "interp": True, "optimize": False, "check": "nan",
     "path": "checked.anvil"},
    {"name": "check_inf", "source": CHECK_INF, "interp": True, "optimize": False, "check": "nan",
     "path": "checked.anvil"},
    {"name": "check_inf_traced", "source": CHECK_INF, "interp": True, "optimize": False, "check": "inf",
     "path": "checked.anvil"},
    {"name": "check_healthy", "source": CHECK_HEALTHY, "interp": True, "optimize": False, "check": "inf",
     "path": "checked.anvil"},
    # the reference's CUDA backend test cases as programs
    {"name": "greet", "source": GREET, "interp": True},
    {"name": "logreg", "source": LOGREG, "interp": True, "keep": ["w", "c"]},
    {"name": "attention_fit", "source": ATTENTION_FIT, "interp": True, "keep": ["A", "O"]},
    {"name": "split", "source": SPLIT, "interp": True},
    {"name": "scatter", "source": SCATTER, "interp": True},
    {"name": "bounds", "source": BOUNDS},
    {"name": "gather_oob", "source": GATHER_OOB},
    {"name": "assert_fail", "source": ASSERT_FAIL},
    {"name": "save_load", "source": SAVE_LOAD},
    {"name": "integers", "source": INTEGERS, "interp": True},
    {"name": "formats", "source": FORMATS, "interp": True},
    {"name": "control", "source": CONTROL, "interp": True},
    {"name": "products", "source": PRODUCTS, "interp": True},
    {"name": "mnist_like", "source": MNIST_LIKE, "interp": True, "keep": C1_KEEP},
    # the run-time calls: data files of every kind, save_npy (the bytes written are kept), nonzero,
    # input from a scripted stdin, checkpoints written by the reference and read back
    {"name": "files", "source": FILES, "interp": True, "files": ["OUT_w2.npy", "OUT_marks.npy"]},
    {"name": "picks", "source": PICKS, "interp": True, "stdin": PICKS_STDIN},
    {"name": "ckpt_write", "source": CKPT_WRITE, "interp": True, "files": ["OUT_pair.ckpt"],
     "publish": {"OUT_pair.ckpt": "pair.ckpt"}},
    {"name": "ckpt_read", "source": CKPT_READ, "interp": True},
    # plain stores through an index with repeated targets: the last write wins, in domain order
    {"name": "serial", "source": SERIAL, "interp": True, "keep": ["slots", "dst"]},
    # show(): one glyph per element, "?" for values past the glyphs
    {"name": "board", "source": BOARD, "interp": True},
    # device-drawn random numbers, printed (uniforms also as the integers u·2²² and g·2²⁴, their exact
    # bits) and kept, bit for bit; printed last, so every tensor keeps its memory to the end
    {"name": "draws", "source": DRAWS, "interp": True, "keep": ["u", "k", "b", "m"]},
    # north-star tolerances at full size: C2 after 100 steps (every parameter), the first step's loss
    # of C2, C4 and C5 to 7 digits, and C4 at T = 256
    {"name": "c2_full100", "source": C2, "consts": {"STEPS": 100}, "interp": True, "keep": C2_KEEP[:6]},
    {"name": "c4_t256_2", "source": C4, "consts": {"STEPS": 2, "T": 256}, "interp": True,
     "keep": ["net.layers.0.Wqkv", "net.layers.3.ff_in.W", "net.head.W", "net.head.b"]},
    {"name": "c5_step1", "source": C5, "consts": {"STEPS": 1}, "interp": True},
    # C5's first convolution with 12 output channels: the outer-product schedule's row groups of 8
    # end in a partial group of 4
    {"name": "c5_conv12", "source": C5, "consts": {"STEPS": 2, "NB": 32, "C1": 12, "C2": 16, "HID": 32},
     "interp": True, "keep": ["net.c1.W", "net.c1.b", "net.c2.W", "net.fc1.W"]},
    # C4 with five 32-row tiles per head: the training attention's workgroups take the tile pairs
    # (0, 4), (1, 3) and the middle tile 2 alone, with all of a pair's key tiles staged at once
    {"name": "c4_t160", "source": C4,
     "consts": {"STEPS": 2, "BATCH": 2, "T": 160, "D": 128, "HEADS": 2, "LAYERS": 1}, "interp": True,
     "own_process": True, "keep": ["net.tok", "net.layers.0.Wqkv", "net.layers.0.Wout", "net.head.W"]},
    # a `+=` into table rows picked by an index array at sizes the C4 fixtures do not reach: more
    # columns than a workgroup has lanes, positions not a multiple of 256, an odd number of rows
    {"name": "scatter_rows", "interp": True, "own_process": True, "keep": ["G", "S"], "source": """
tok: i32[9, 111] ~ randint(0, 7)
X: [9, 111, 300] ~ normal(0, 1)
G: [7, 300] = 0.0
G[tok[n, t], d] += X[n, t, d]
S: [7, 300] = 0.0
S[tok[n, t], d] += X[n, t, d] * 2.0 - 1.0
print(G[0:2])
print(S[5:7])
"""},
    {"name": "argpick", "source": ARGPICK, "interp": True, "own_process": True},
    # attention chains the fused training attention must leave to the generated kernels (IR only):
    # queries and keys read from the same columns of qkv (their gradients add into one slice), and
    # a projection with a fourth slice that no head reads (its gradient is 0, written by no launch);
    # the generated kernels then run against the reference interpreter's vectors
    {"name": "attn_same_qk", "own_process": True, "interp": True, "keep": ["net.layers.0.Wqkv"],
     "source": C4.replace("qkv[n, u, 1, h, c]", "qkv[n, u, 0, h, c]"), "consts": C4_MID},
    {"name": "attn_four_slices", "own_process": True, "interp": True, "keep": ["net.layers.0.Wqkv"],
     "source": C4.replace("[D, 3 * D]", "[D, 4 * D]").replace("reshape(-1, T, 3, HEADS, DH)",
                                                               "reshape(-1, T, 4, HEADS, DH)"),
     "consts": C4_MID},
    # a row block (one workgroup per row) whose second stage adds into rows that a kernel before the
    # chain wrote (y, 256 elements a row): the stage must read the prior writer's values
    {"name": "rowblock_prior", "interp": True, "own_process": True, "source": """
X: [256, 256] ~ normal(0, 1)
fn f(x: [n, m]):
    y = x * 2.0
    s[i] = sum y[i, j]
    y[i, j] -= s[i] / 256.0
    t[i, q] = sum y[i, 4 * q + c] where c < 4
    return t
for step in range(2):
    r = f(X)
    print(r[0:2, 0:3])
    print(sum(r))
"""},
    # C4 and C5 over their whole BASELINE runs (200 Adam steps at T = 64; 300 SGD steps), the loss
    # printed every 20 (30) steps along the way and the trained weights kept
    {"name": "c4_full200", "own_process": True, "interp": True,
     "source": C4.replace('    if step == 0:\n        print("step 1 loss {loss:.6e}")',
                          '    if step == 0 or step % 20 == 19:\n        print("step {step + 1} loss {loss:.6e}")'),
     "keep": ["net.layers.0.Wqkv", "net.layers.3.ff_in.W", "net.head.W", "net.head.b"]},
    {"name": "c5_full300", "own_process": True, "interp": True,
     "source": C5.replace('    if step == 0:\n        print("step 1 loss {loss:.6e}")',
                          '    if step == 0 or step % 30 == 29:\n        print("step {step + 1} loss {loss:.6e}")'),
     "keep": ["net.c1.W", "net.c1.b", "net.c2.W", "net.c2.b", "net.fc1.W", "net.fc2.W"]},
] + [
    # anvil.function's surface as the reference's tests/test_pyapi.py:32-134 uses it, one lowering
    # (pyapi.lower) per argument signature: an i32 argument and a number passed as a compile-time
    # constant (two versions), a constant used as a shape, a loss-and-gradient tuple with a scalar,
    # a scalar result, a compile-time result beside a tensor one, a function that assigns into its
    # argument, a float64 / transposed argument, a NumPy scalar argument (threads call it), causal
    # attention
    {"name": f"fn_{name}", "source": src, "interp": True, "own_process": True, "function": {"name": fname, "args": args}}
    for name, src, fname, args in [
        ("pick", "fn pick(x: [n, d], idx: i32[k], scale) = x[idx] * scale\n", "pick",
         [([10, 3], "f32"), ([3], "i32"), ("const", "2.0")]),
        ("pick_half", "fn pick(x: [n, d], idx: i32[k], scale) = x[idx] * scale\n", "pick",
         [([10, 3], "f32"), ([2], "i32"), ("const", "0.5")]),
        ("shifted", "fn shifted(x: [n], k):\n    y[i] = x[i + k] where i < n - k\n    return y\n", "shifted",
         [([6], "f32"), ("const", "2")]),
        ("loss_grad", "fn loss_and_grad(w: [d], x: [n, d], y: [n]):\n    loss = mean((x @ w - y) ** 2)\n"
                      "    return loss, grad(loss, w)\n", "loss_and_grad", [([5], "f32"), ([32, 5], "f32"), ([32], "f32")]),
        ("total", "fn total(x) = sum(x)\n", "total", [([10], "f32")]),
        ("sizes", "fn sizes(x: [n, d]):\n    return n * d, sum(x)\n", "sizes", [([3, 4], "f32")]),
        ("keeps_args", "fn f(x: [n]):\n    x[0] = 1.0\n    return x * 2\n", "f", [([4], "f32")]),
        ("double", "fn double(x) = x * 2\n", "double", [([4, 3], "f32")]),
        # a NumPy scalar argument arrives as a [1] tensor (pyapi.arguments: np.ascontiguousarray)
        ("scaled", "fn scaled(x, s) = x * s\n", "scaled", [([1000], "f32"), ([1], "f32")]),
        ("causal", "fn attention(q: [b, t, d], k: [b, t, d], v: [b, t, d]):\n"
                   "    s[n, i, j] = sum q[n, i, c] * k[n, j, c] / sqrt(d) + (0.0 if j <= i else -1e9)\n"
                   "    return softmax(s) @ v\n", "attention", [([3, 7, 4], "f32")] * 3),
    ]
]
