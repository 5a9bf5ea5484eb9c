/*
 * cfg.c -- darknet-style .cfg files -> an_network.  Follows the reference's
 * ConfigFile (ConfigFile.c:12-208, INI groups and key=value pairs, '#' and
 * ';' comments) and the defaults of NetworkFactory (paths relative to
 * /root/reference/src/com/ai/dnn/):
 *   [net]            parseNetOption NetworkFactory.c:671-700
 *                    batch=1 learning_rate=.001 momentum=.9 decay=.0001
 *                    subdivisions=1 (batch /= subdivisions)
 *                    policy=constant burn_in=0 power=4 max_batches=0
 *                    (NetworkFactory.c:676,763-823): step: step=1 scale=1;
 *                    steps: steps=, scales= (comma lists, required);
 *                    exp: gamma=1; sigmoid: gamma=1 step=1; unknown
 *                    policy names fall back to constant (ConfigFile.c:159-168)
 *   [convolutional]  createConvolutional NetworkFactory.c:77-103
 *                    filters=1 size=1 stride=1 pad=0 padding=0
 *                    (pad=1 -> padding=size/2) activation=logistic
 *                    batch_normalize=0
 *   [connected]      not built by the reference (no CONNECTED case in
 *                    createLayer, NetworkFactory.c:615-654); darknet's keys:
 *                    output=1 activation=logistic batch_normalize=0
 *   [maxpool]        createMaxPool NetworkFactory.c:543-548
 *                    stride=1 size=stride padding=size-1
 *   [avgpool]        createAvgPool NetworkFactory.c:572-584
 *   [dropout]        createDropoutLayer NetworkFactory.c:328-329  probability=.2
 *   [softmax]        createSoftMax NetworkFactory.c:586-601 groups=1 temperature=1
 * Every layer section also takes the options of createLayer /
 * createNetwork (NetworkFactory.c:656-663, 926-935) that the CPU path acts
 * on: stopbackward, onlyforward, dontload, dontloadscales, learning_rate
 * (a float scale of the layer's rate) and, for [convolutional], flipped.
 * Keys the reference reads whose non-default values change its CPU
 * training step but this build does not implement (groups, dilation,
 * xnor, binary, bin_output, antialiasing, cbn, deformable sway / rotate /
 * stretch, assisted_excitation, share_index, maxpool_depth, dropblock, softmax spatial / noloss / tree, [net]
 * time_steps) are rejected with a message.  Keys the reference reads but
 * its CPU path never acts on are accepted; keys it does not read are
 * reported as unused (darknet's behaviour).
 */
#include "aetcnn_net.h"

#include <ctype.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define CFG_MAX_KV 64

typedef struct {
    char name[64];
    int nkv;
    char key[CFG_MAX_KV][64];
    char val[CFG_MAX_KV][128];
} cfg_group;

static char *trim(char *s)
{
    while (*s && isspace((unsigned char)*s)) ++s;
    char *e = s + strlen(s);
    while (e > s && isspace((unsigned char)e[-1])) *--e = 0;
    return s;
}

static const char *find(const cfg_group *g, const char *k)
{
    for (int i = 0; i < g->nkv; ++i)
        if (!strcmp(g->key[i], k)) return g->val[i];
    return NULL;
}

static int geti(const cfg_group *g, const char *k, int def)
{
    const char *v = find(g, k);
    return v ? atoi(v) : def;
}

static float getf(const cfg_group *g, const char *k, float def)
{
    const char *v = find(g, k);
    return v ? (float)atof(v) : def;
}

static int activation_id(const char *s)
{
    /* Activation.getActivation (Activation.c:104-120) names */
    if (!strcmp(s, "logistic")) return ACH_LOGISTIC;
    if (!strcmp(s, "relu")) return ACH_RELU;
    if (!strcmp(s, "linear")) return ACH_LINEAR;
    if (!strcmp(s, "leaky")) return ACH_LEAKY;
    return -1;
}

static int read_groups(const char *path, cfg_group **out, int *count)
{
    FILE *f = fopen(path, "r");
    if (!f) {
        fprintf(stderr, "an_parse_cfg: cannot open %s\n", path);
        return -1;
    }
    int cap = 16, n = 0;
    cfg_group *gs = (cfg_group *)calloc(cap, sizeof(cfg_group));
    if (!gs) {
        fclose(f);
        return -1;
    }
    char line[512];
    int lineno = 0;
    while (fgets(line, sizeof(line), f)) {
        ++lineno;
        char *s = trim(line);
        if (!*s || *s == '#' || *s == ';') continue;
        if (*s == '[') {
            char *e = strchr(s, ']');
            if (!e) goto bad;
            *e = 0;
            if (n == cap) {
                cfg_group *ng = (cfg_group *)realloc(gs, sizeof(cfg_group) * cap * 2);
                if (!ng) {
                    fprintf(stderr, "an_parse_cfg: out of host memory\n");
                    fclose(f);
                    free(gs);
                    return -1;
                }
                gs = ng;
                cap *= 2;
            }
            memset(&gs[n], 0, sizeof(cfg_group));
            snprintf(gs[n].name, sizeof(gs[n].name), "%s", trim(s + 1));
            ++n;
            continue;
        }
        char *eq = strchr(s, '=');
        if (!eq || n == 0) goto bad;
        *eq = 0;
        cfg_group *g = &gs[n - 1];
        if (g->nkv == CFG_MAX_KV) goto bad;
        snprintf(g->key[g->nkv], sizeof(g->key[0]), "%s", trim(s));
        snprintf(g->val[g->nkv], sizeof(g->val[0]), "%s", trim(eq + 1));
        g->nkv++;
    }
    fclose(f);
    *out = gs;
    *count = n;
    return 0;
bad:
    fprintf(stderr, "an_parse_cfg: %s:%d: cannot parse line\n", path, lineno);
    fclose(f);
    free(gs);
    return -1;
}

static int unsupported(const cfg_group *g, const char *key, int def)
{
    const char *v = find(g, key);
    if (v && atoi(v) != def) {
        fprintf(stderr, "an_parse_cfg: [%s] %s=%s is not supported\n", g->name, key, v);
        return 1;
    }
    return 0;
}

/* a key whose mere presence asks for something not built */
static int present_unsupported(const cfg_group *g, const char *key)
{
    const char *v = find(g, key);
    if (v) {
        fprintf(stderr, "an_parse_cfg: [%s] %s=%s is not supported\n", g->name, key, v);
        return 1;
    }
    return 0;
}

/* The keys the reference reads in each section (NetworkFactory.c:77-173,
 * 328-340, 543-601, 656-663, 671-823, 926-935); any other key is reported
 * as unused, as darknet does.                                              */
static const char *const NET_KEYS[] = {
    "max_batches", "batch", "learning_rate", "learning_rate_min", "sgdr_cycle", "sgdr_mult",
    "momentum", "decay", "subdivisions", "time_steps", "track", "augment_speed",
    "sequential_subdivisions", "try_fix_nan", "weights_reject_freq", "equidistant_point",
    "badlabels_rejection_percentage", "num_sigmas_reject_badlabels", "ema_alpha",
    "use_cuda_graph", "loss_scale", "dynamic_minibatch", "optimized_memory",
    "workspace_size_limit_MB", "adam", "B1", "B2", "eps", "height", "width", "channels",
    "inputs", "max_crop", "min_crop", "flip", "blur", "gaussian_noise", "mixup", "cutmix",
    "mosaic", "letter_box", "mosaic_bound", "contrastive", "contrastive_jit_flip",
    "contrastive_color", "unsupervised", "label_smooth_eps", "resize_step", "attention",
    "adversarial_lr", "max_chart_loss", "angle", "aspect", "saturation", "exposure", "hue",
    "power", "policy", "burn_in", "step", "scale", "steps", "scales", "seq_scales", "gamma",
    NULL};
static const char *const LAYER_KEYS[] = { /* createLayer + createNetwork, every layer */
    "truth", "onlyforward", "stopbackward", "dontsave", "dontload", "numload",
    "dontloadscales", "learning_rate", "smooth", "clip", "dont_update", "burnin_update",
    "train_only_bn", NULL};
static const char *const CONV_KEYS[] = {
    "filters", "groups", "size", "stride", "stride_x", "stride_y", "dilation", "antialiasing",
    "pad", "padding", "activation", "assisted_excitation", "share_index", "batch_normalize",
    "cbn", "binary", "xnor", "bin_output", "sway", "rotate", "stretch", "stretch_sway",
    "flipped", "dot", "angle", "grad_centr", "reverse", "coordconv", "stream", "wait_stream",
    NULL};
static const char *const CONN_KEYS[] = {"output", "activation", "batch_normalize", NULL};
static const char *const MAXPOOL_KEYS[] = {
    "stride", "stride_x", "stride_y", "size", "padding", "maxpool_depth", "out_channels",
    "antialiasing", "maxpool_zero_nonmax", NULL};
static const char *const DROPOUT_KEYS[] = {
    "probability", "dropblock", "dropblock_size_rel", "dropblock_size_abs", NULL};
static const char *const SOFTMAX_KEYS[] = {
    "groups", "temperature", "spatial", "noloss", "tree", NULL};
static const char *const NO_KEYS[] = {NULL};

static int in_list(const char *const *l, const char *k)
{
    for (; *l; ++l)
        if (!strcmp(*l, k)) return 1;
    return 0;
}

static void report_unused(const cfg_group *g, const char *const *own, int layer)
{
    for (int i = 0; i < g->nkv; ++i)
        if (!in_list(own, g->key[i]) && !(layer && in_list(LAYER_KEYS, g->key[i])))
            fprintf(stderr, "an_parse_cfg: unused field [%s] %s=%s\n", g->name, g->key[i],
                    g->val[i]);
}

/* stride_x / stride_y as createConvolutional / createMaxPool resolve them
 * (NetworkFactory.c:83-93, 545-546): a convolution's missing or nonpositive
 * value falls back to stride, a pool's missing one.  Returns 0, or -1 for a
 * stride below 1 (which the layer constructors reject).                   */
static int layer_strides(const cfg_group *g, int conv, int *sx, int *sy)
{
    const int stride = geti(g, "stride", 1);
    *sx = geti(g, "stride_x", conv ? -1 : stride);
    *sy = geti(g, "stride_y", conv ? -1 : stride);
    if (conv && (*sx < 1 || *sy < 1)) {
        if (*sx < 1) *sx = stride;
        if (*sy < 1) *sy = stride;
    }
    if (*sx < 1 || *sy < 1) {
        fprintf(stderr, "an_parse_cfg: [%s] stride_x=%d stride_y=%d\n", g->name, *sx, *sy);
        return -1;
    }
    return 0;
}

/* the createLayer / createNetwork options of layer `idx` */
static int layer_options(an_network *net, int idx, const cfg_group *g, int conv)
{
    an_layer_options o;
    o.stopbackward = geti(g, "stopbackward", 0);
    o.onlyforward = geti(g, "onlyforward", 0);
    o.dontload = geti(g, "dontload", 0);
    o.dontloadscales = geti(g, "dontloadscales", 0);
    o.flipped = conv ? geti(g, "flipped", 0) : 0;
    o.learning_rate_scale = getf(g, "learning_rate", 1.f);
    if (an_set_layer_options(net, idx, &o) != ACH_OK) {
        fprintf(stderr, "an_parse_cfg: [%s] invalid layer options\n", g->name);
        return -1;
    }
    return 0;
}

/* a comma list of up to `cap` numbers ('#' ends it); returns the count or -1 */
static int parse_list(const char *v, int cap, int *iv, float *fv)
{
    int n = 0;
    const char *p = v;
    while (*p && *p != '#') {
        if (n == cap) return -1;
        char *end;
        const double x = strtod(p, &end);
        if (end == p) return -1;
        if (iv) iv[n] = (int)x;
        if (fv) fv[n] = (float)x;
        ++n;
        p = end;
        while (isspace((unsigned char)*p)) ++p;
        if (*p == ',') ++p;
        else if (*p && *p != '#') return -1;
    }
    return n;
}

#define CFG_MAX_STEPS 64

/* parseNetOption's policy keys (NetworkFactory.c:763-823) */
static int parse_policy(an_network *net, const cfg_group *g)
{
    static const struct { const char *name; int id; } names[] = {
        {"random", AN_POLICY_RANDOM}, {"poly", AN_POLICY_POLY},
        {"constant", AN_POLICY_CONSTANT}, {"step", AN_POLICY_STEP},
        {"exp", AN_POLICY_EXP}, {"sigmoid", AN_POLICY_SIG}, {"steps", AN_POLICY_STEPS}};
    const char *ps = find(g, "policy");
    int policy = AN_POLICY_CONSTANT;
    if (ps) {
        int found = 0;
        for (size_t i = 0; i < sizeof(names) / sizeof(names[0]); ++i)
            if (!strcmp(ps, names[i].name)) {
                policy = names[i].id;
                found = 1;
            }
        if (!found) fprintf(stderr, "Couldn't find policy %s, going with constant\n", ps);
    }
    const int burn_in = geti(g, "burn_in", 0);
    const float power = getf(g, "power", 4.f);
    const int max_batches = geti(g, "max_batches", 0);
    float gamma = 1.f, scale = 1.f;
    int step = 1, nsteps = 0;
    int steps[CFG_MAX_STEPS];
    float scales[CFG_MAX_STEPS];
    if (policy == AN_POLICY_STEP) {
        step = geti(g, "step", 1);
        scale = getf(g, "scale", 1.f);
    } else if (policy == AN_POLICY_STEPS) {
        const char *l = find(g, "steps"), *p = find(g, "scales");
        if (!l || !p) {
            fprintf(stderr, "an_parse_cfg: STEPS policy must have steps and scales\n");
            return -1;
        }
        nsteps = parse_list(l, CFG_MAX_STEPS, steps, NULL);
        if (nsteps <= 0 || parse_list(p, CFG_MAX_STEPS, NULL, scales) != nsteps) {
            fprintf(stderr, "an_parse_cfg: steps and scales need the same count of numbers\n");
            return -1;
        }
    } else if (policy == AN_POLICY_EXP) {
        gamma = getf(g, "gamma", 1.f);
    } else if (policy == AN_POLICY_SIG) {
        gamma = getf(g, "gamma", 1.f);
        step = geti(g, "step", 1);
    }
    if (an_set_policy(net, policy, burn_in, power, gamma, scale, step, max_batches, nsteps,
                      steps, scales)) {
        fprintf(stderr, "an_parse_cfg: invalid learning-rate policy settings\n");
        return -1;
    }
    return 0;
}

an_network *an_parse_cfg_unfinalized(const char *path)
{
    cfg_group *gs = NULL;
    int ng = 0;
    if (!path || read_groups(path, &gs, &ng)) return NULL;
    an_network *net = NULL;
    if (ng == 0 || (strcmp(gs[0].name, "net") && strcmp(gs[0].name, "network"))) {
        fprintf(stderr, "an_parse_cfg: first section must be [net] or [network]\n");
        goto fail;
    }
    {
        const cfg_group *g = &gs[0];
        int batch = geti(g, "batch", 1);
        const int subdivs = geti(g, "subdivisions", 1);
        if (subdivs <= 0) goto fail;
        batch /= subdivs;
        if (batch < 1) batch = 1;
        if (unsupported(g, "time_steps", 1)) goto fail;
        const int h = geti(g, "height", 0), w = geti(g, "width", 0), c = geti(g, "channels", 0);
        if (find(g, "inputs") && geti(g, "inputs", 0) != h * w * c) {
            fprintf(stderr, "an_parse_cfg: [net] inputs must equal height*width*channels\n");
            goto fail;
        }
        report_unused(g, NET_KEYS, 0);
        net = an_network_create(batch, h, w, c);
        if (!net) {
            fprintf(stderr, "an_parse_cfg: [net] needs height, width and channels\n");
            goto fail;
        }
        an_set_hyper(net, getf(g, "learning_rate", .001f), getf(g, "momentum", .9f),
                     getf(g, "decay", .0001f));
        if (an_set_subdivisions(net, subdivs) || parse_policy(net, g)) goto fail;
    }
    for (int i = 1; i < ng; ++i) {
        const cfg_group *g = &gs[i];
        int rc;
        int conv = 0;
        if (!strcmp(g->name, "convolutional") || !strcmp(g->name, "conv")) {
            const int size = geti(g, "size", 1);
            conv = 1;
            report_unused(g, CONV_KEYS, 1);
            /* dilation is forced to 1 for 1x1 filters (NetworkFactory.c:97-98) */
            if (unsupported(g, "groups", 1) || (size != 1 && unsupported(g, "dilation", 1)) ||
                unsupported(g, "xnor", 0) || unsupported(g, "binary", 0) ||
                unsupported(g, "bin_output", 0) || unsupported(g, "antialiasing", 0) ||
                unsupported(g, "cbn", 0) || unsupported(g, "sway", 0) ||
                unsupported(g, "rotate", 0) || unsupported(g, "stretch", 0) ||
                unsupported(g, "stretch_sway", 0) || unsupported(g, "assisted_excitation", 0) ||
                present_unsupported(g, "share_index"))
                goto fail;
            int sx, sy;
            if (layer_strides(g, 1, &sx, &sy)) goto fail;
            int padding = geti(g, "padding", 0);
            if (geti(g, "pad", 0)) padding = size / 2;
            const char *an = find(g, "activation");
            const int act = activation_id(an ? an : "logistic");
            if (act < 0) {
                fprintf(stderr, "an_parse_cfg: activation %s is not supported\n", an);
                goto fail;
            }
            rc = an_add_convolutional_xy(net, geti(g, "filters", 1), size, sx, sy, padding, act,
                                         geti(g, "batch_normalize", 0));
        } else if (!strcmp(g->name, "connected") || !strcmp(g->name, "conn")) {
            report_unused(g, CONN_KEYS, 1);
            const char *an = find(g, "activation");
            const int act = activation_id(an ? an : "logistic");
            if (act < 0) {
                fprintf(stderr, "an_parse_cfg: activation %s is not supported\n", an);
                goto fail;
            }
            rc = an_add_connected(net, geti(g, "output", 1), act, geti(g, "batch_normalize", 0));
        } else if (!strcmp(g->name, "maxpool") || !strcmp(g->name, "max")) {
            report_unused(g, MAXPOOL_KEYS, 1);
            if (unsupported(g, "maxpool_depth", 0) || unsupported(g, "antialiasing", 0))
                goto fail;
            int sx, sy;
            if (layer_strides(g, 0, &sx, &sy)) goto fail;
            /* the size defaults to the stride key, not the resolved strides */
            const int size = geti(g, "size", geti(g, "stride", 1));
            rc = an_add_maxpool_xy(net, size, sx, sy, geti(g, "padding", size - 1));
        } else if (!strcmp(g->name, "avgpool") || !strcmp(g->name, "avg")) {
            report_unused(g, NO_KEYS, 1);
            rc = an_add_avgpool(net);
        } else if (!strcmp(g->name, "dropout")) {
            report_unused(g, DROPOUT_KEYS, 1);
            if (unsupported(g, "dropblock", 0)) goto fail;
            rc = an_add_dropout(net, getf(g, "probability", .2f));
        } else if (!strcmp(g->name, "softmax") || !strcmp(g->name, "soft")) {
            report_unused(g, SOFTMAX_KEYS, 1);
            if (unsupported(g, "spatial", 0) || unsupported(g, "noloss", 0) ||
                present_unsupported(g, "tree"))
                goto fail;
            rc = an_add_softmax(net, geti(g, "groups", 1), getf(g, "temperature", 1.f));
        } else {
            fprintf(stderr, "an_parse_cfg: layer type [%s] is not supported\n", g->name);
            goto fail;
        }
        if (rc < 0) {
            fprintf(stderr, "an_parse_cfg: cannot build [%s] (section %d): code %d\n", g->name,
                    i, rc);
            goto fail;
        }
        if (layer_options(net, rc, g, conv)) goto fail;
    }
    free(gs);
    return net;
fail:
    free(gs);
    an_free(net);
    return NULL;
}

an_network *an_parse_cfg(const char *path)
{
    an_network *net = an_parse_cfg_unfinalized(path);
    if (!net) return NULL;
    if (an_finalize(net) != ACH_OK) {
        fprintf(stderr, "an_parse_cfg: finalize failed\n");
        an_free(net);
        return NULL;
    }
    return net;
}

/* The augmentation keys of [net] (parseNetOption, NetworkFactory.c:727-762:
 * max_crop = width*2, min_crop = width, flip = 1, angle = 0, aspect = 1,
 * saturation = 1, exposure = 1, hue = 0; label_smooth_eps = 0) read as the
 * reference reads them; the input pipeline applies them (an_augment_image). */
int an_cfg_augment(const char *path, an_augment *a, float *label_smooth_eps)
{
    cfg_group *gs = NULL;
    int ng = 0;
    if (!path || !a || read_groups(path, &gs, &ng)) return ACH_EINVAL;
    if (ng == 0 || (strcmp(gs[0].name, "net") && strcmp(gs[0].name, "network"))) {
        free(gs);
        return ACH_EINVAL;
    }
    const cfg_group *g = &gs[0];
    const int w = geti(g, "width", 0);
    an_augment_defaults(a, w);
    a->max_crop = geti(g, "max_crop", w * 2);
    a->min_crop = geti(g, "min_crop", w);
    a->flip = geti(g, "flip", 1);
    a->angle = getf(g, "angle", 0.f);
    a->aspect = getf(g, "aspect", 1.f);
    a->saturation = getf(g, "saturation", 1.f);
    a->exposure = getf(g, "exposure", 1.f);
    a->hue = getf(g, "hue", 0.f);
    if (label_smooth_eps) *label_smooth_eps = getf(g, "label_smooth_eps", 0.f);
    free(gs);
    return ACH_OK;
}
